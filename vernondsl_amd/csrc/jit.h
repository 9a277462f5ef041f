// Run-time compilation of kernels specialised for one program (host side), shared by the op
// classes that compile per program: map chains (map_chain.hip) and per-pixel programs
// (pixel_prog.hip).  A source is compiled once per device with hiprtc, with the library's own
// device flags and its embedded headers (vdsl.h, fmath.h, mapchain_kern.h, pixprog_kern.h), and
// loaded as a module; the source text, which names every entry point, is the cache key.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <string>

namespace vdsl {

struct JitKernels {
  hipModule_t mod = nullptr;
  hipFunction_t fn[2] = {nullptr, nullptr};  // the entry points, in the order they were named
  bool failed = false;
};

struct JitCounters {
  std::atomic<int64_t> compiles{0}, failures{0};
};

// The kernels `entries[0 .. n_entries)` (at most 2) of `src` on device `ordinal`.  Compiles and
// loads them on first use unless `lookup_only` (then VDSL_ERR_UNSUPPORTED if they are not there
// yet).  A source whose compilation failed is not retried: the call fails again with
// VDSL_ERR_DEVICE.  `what` names the op class in error messages.
int jit_kernels(int ordinal, const std::string& src, const char* const* entries, int n_entries, bool lookup_only,
                JitCounters& ctr, const char* what, const JitKernels** out);

}  // namespace vdsl
