// Op class 4: dense bf16 x bf16 -> f32-accumulate GEMM on gfx950 MFMA, with fused epilogues.
//
// No reference code (the north-star op class: the dense matmuls of the MLP graph, forward and
// autodiff-generated backward).
//
// Native layout "NT": C[m][n] = sum_k A[m][k] * B[n][k], both operands K-contiguous (B is a
// weight in [out][in] form).  The other layouts are reduced to it by transposing the strided
// operand into caller-provided workspace first (vdsl_gemm_bf16_workspace_bytes).
//
// Tiling: a 256-lane block computes a 128x128 tile of C; its 4 waves form a 2x2 grid of 64x64
// wave tiles, each a 2x2 grid of v_mfma_f32_32x32x16_bf16 accumulators (64 f32 per lane).  K
// advances 64 at a time through LDS (A and B tiles [128][64+8] bf16; the 8-element pad staggers
// rows across banks for the 16-byte fragment reads).  The next K tile's global loads are
// issued into registers before the MFMAs of the current one, so HBM latency hides behind
// matrix work.  Block ids are remapped so that blocks dispatched to the same XCD (ids congruent
// mod 8) take neighbouring tiles and share A/B rows in that XCD's L2.
//
// MFMA operand layout used (32x32x16 bf16, wave64): lane l supplies A[row = l%32][k = 8*(l/32)
// .. +7] and B[col = l%32][k = 8*(l/32) .. +7]; accumulator element r of lane l is
// C[row = 8*(r/4) + 4*(l/32) + r%4][col = l%32].

#include "common.h"

namespace vdsl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Defined in layout.hip.
int launch_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int dtype, hipStream_t s);

namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;

// 0.5 v (1 + erf(v / sqrt2)) written as 0.5 v erfc(-v / sqrt2): no cancellation for v < 0.
__device__ __forceinline__ float gelu_f(float v) { return 0.5f * v * erfcf(-v * 0.7071067811865476f); }

__device__ __forceinline__ int remap_xcd(int b, int nb) {
  // Hardware dispatches block b to XCD b % 8.  Give the blocks of one XCD a contiguous range of
  // tile ids (when the grid divides evenly; otherwise keep the identity order).
  if (nb % 8) return b;
  return (b % 8) * (nb / 8) + (b / 8);
}

template <int EPI, int CT, bool PRE>
__global__ __launch_bounds__(256, 2) void gemm_bf16_nt(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                       void* __restrict__ C, float* __restrict__ pre, int M, int N,
                                                       int K) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int tiles_n = (N + BN - 1) / BN;
  const int nb = gridDim.x;
  const int t = remap_xcd(blockIdx.x, nb);
  // Tile order: groups of 8 tile-rows walked column by column, so consecutive tiles reuse B.
  const int tiles_m = (M + BM - 1) / BM;
  constexpr int G = 8;
  const int group = t / (G * tiles_n);
  const int first_m = group * G;
  const int gsize = min(G, tiles_m - first_m);
  const int in_group = t - group * G * tiles_n;
  const int tile_m = first_m + in_group % gsize;
  const int tile_n = in_group / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Each lane moves 4 16-byte chunks of A and of B per K tile: chunk c = tid + 256*i covers
  // row c/8, k-chunk c%8 (8 lanes read one 128-byte row segment).
  uint4 ra[4], rb[4];
  auto load_tiles = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3;
      const int k = kt * BK + (c & 7) * 8;
      const int gm = m0 + row, gn = n0 + row;
      ra[i] = (gm < M && k < K) ? *reinterpret_cast<const uint4*>(A + static_cast<size_t>(gm) * K + k) : make_uint4(0, 0, 0, 0);
      rb[i] = (gn < N && k < K) ? *reinterpret_cast<const uint4*>(B + static_cast<size_t>(gn) * K + k) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3;
      const int kc = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&As[row * LDK + kc]) = ra[i];
      *reinterpret_cast<uint4*>(&Bs[row * LDK + kc]) = rb[i];
    }
  };

  const int nk = (K + BK - 1) / BK;
  load_tiles(0);
  store_tiles();
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_tiles(kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const bf16x8*>(&As[(wm * 64 + i * 32 + frag_row) * LDK + kk + frag_k]);
        b[i] = *reinterpret_cast<const bf16x8*>(&Bs[(wn * 64 + i * 32 + frag_row) * LDK + kk + frag_k]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (kt + 1 < nk) {
      store_tiles();
      __syncthreads();
    }
  }

  // Epilogue.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int col = n0 + wn * 64 + j * 32 + (lane & 31);
        if (row < M && col < N) {
          const float v = acc[i][j][r];
          const size_t o = static_cast<size_t>(row) * N + col;
          if (PRE) pre[o] = v;
          float y = v;
          if (EPI == VDSL_EPI_GELU) y = gelu_f(v);
          else if (EPI == VDSL_EPI_RELU) y = v > 0.0f ? v : 0.0f;
          if (CT == VDSL_F32) static_cast<float*>(C)[o] = y;
          else static_cast<uint16_t*>(C)[o] = f32_to_bf16(y);
        }
      }
}

// Any K (including K % 8 != 0): one lane per output, f32 accumulate in k order.
template <int EPI, int CT, bool PRE>
__global__ __launch_bounds__(256) void gemm_bf16_nt_simple(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                           void* __restrict__ C, float* __restrict__ pre, int M, int N,
                                                           int K) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(M) * N) return;
  const int row = static_cast<int>(idx / N), col = static_cast<int>(idx % N);
  float v = 0.0f;
  for (int k = 0; k < K; ++k)
    v = __builtin_fmaf(bf16_to_f32(A[static_cast<size_t>(row) * K + k]), bf16_to_f32(B[static_cast<size_t>(col) * K + k]), v);
  if (PRE) pre[idx] = v;
  float y = v;
  if (EPI == VDSL_EPI_GELU) y = gelu_f(v);
  else if (EPI == VDSL_EPI_RELU) y = v > 0.0f ? v : 0.0f;
  if (CT == VDSL_F32) static_cast<float*>(C)[idx] = y;
  else static_cast<uint16_t*>(C)[idx] = f32_to_bf16(y);
}

template <int EPI, int CT, bool PRE>
int launch_nt3(const uint16_t* A, const uint16_t* B, void* C, float* pre, int M, int N, int K, hipStream_t s) {
  if (K % 8 == 0) {
    const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_bf16_nt<EPI, CT, PRE>), dim3(static_cast<unsigned>(tiles)), dim3(256), 0, s, A, B, C, pre, M,
                       N, K);
  } else {
    const int64_t blocks = (static_cast<int64_t>(M) * N + 255) / 256;
    hipLaunchKernelGGL((gemm_bf16_nt_simple<EPI, CT, PRE>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, A, B, C,
                       pre, M, N, K);
  }
  return check_launch("gemm_bf16_nt");
}

template <int EPI, int CT>
int launch_nt2(const uint16_t* A, const uint16_t* B, void* C, float* pre, int M, int N, int K, hipStream_t s) {
  if (pre) return launch_nt3<EPI, CT, true>(A, B, C, pre, M, N, K, s);
  return launch_nt3<EPI, CT, false>(A, B, C, pre, M, N, K, s);
}

template <int EPI>
int launch_nt1(const uint16_t* A, const uint16_t* B, void* C, int ct, float* pre, int M, int N, int K, hipStream_t s) {
  if (ct == VDSL_F32) return launch_nt2<EPI, VDSL_F32>(A, B, C, pre, M, N, K, s);
  return launch_nt2<EPI, VDSL_BF16>(A, B, C, pre, M, N, K, s);
}

size_t workspace_bytes(int ta, int tb, int64_t M, int64_t N, int64_t K) {
  size_t b = 0;
  if (ta) b += static_cast<size_t>(M) * K * 2;
  if (!tb) b += static_cast<size_t>(N) * K * 2;
  return b;
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_gemm_bf16_workspace_bytes(int32_t trans_a, int32_t trans_b, int64_t M, int64_t N, int64_t K,
                                              size_t* bytes) {
  if (!bytes) return fail(VDSL_ERR_INVALID_ARG, "bytes is null");
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  *bytes = workspace_bytes(trans_a != 0, trans_b != 0, M, N, K);
  return VDSL_OK;
}

extern "C" int vdsl_op_gemm_bf16(vdsl_queue q, int32_t trans_a, int32_t trans_b, int64_t M, int64_t N, int64_t K,
                                 vdsl_buffer A, vdsl_buffer B, vdsl_buffer C, int32_t c_dtype, int32_t epilogue,
                                 vdsl_buffer pre_act, vdsl_buffer workspace) {
  VDSL_TRY(enter_queue(q));
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "GEMM extent exceeds 2^31-1");
  if (c_dtype != VDSL_F32 && c_dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "C must be f32 or bf16");
  if (epilogue < VDSL_EPI_NONE || epilogue > VDSL_EPI_RELU) return fail(VDSL_ERR_INVALID_ARG, "unknown epilogue");
  const bool ta = trans_a != 0, tb = trans_b != 0;
  VDSL_TRY(check_buffer(q, A, static_cast<size_t>(M) * K * 2, "A", false));
  VDSL_TRY(check_buffer(q, B, static_cast<size_t>(N) * K * 2, "B", false));
  VDSL_TRY(check_buffer(q, C, static_cast<size_t>(M) * N * dtype_size(c_dtype), "C", true));
  if (pre_act) VDSL_TRY(check_buffer(q, pre_act, static_cast<size_t>(M) * N * 4, "pre_act", true));
  const size_t ws = workspace_bytes(ta, tb, M, N, K);
  if (ws) VDSL_TRY(check_buffer(q, workspace, ws, "workspace", true));
  if (M == 0 || N == 0) return VDSL_OK;

  const uint16_t* a = static_cast<const uint16_t*>(A->ptr);
  const uint16_t* b = static_cast<const uint16_t*>(B->ptr);
  char* w = ws ? static_cast<char*>(workspace->ptr) : nullptr;
  if (ta) {  // A stored [K][M] -> [M][K]
    VDSL_TRY(launch_transpose(a, w, K, M, VDSL_BF16, q->stream));
    a = reinterpret_cast<const uint16_t*>(w);
    w += static_cast<size_t>(M) * K * 2;
  }
  if (!tb) {  // B stored [K][N] -> [N][K]
    VDSL_TRY(launch_transpose(b, w, K, N, VDSL_BF16, q->stream));
    b = reinterpret_cast<const uint16_t*>(w);
  }
  float* pre = pre_act ? static_cast<float*>(pre_act->ptr) : nullptr;
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  switch (epilogue) {
    case VDSL_EPI_GELU: return launch_nt1<VDSL_EPI_GELU>(a, b, C->ptr, c_dtype, pre, m, n, k, q->stream);
    case VDSL_EPI_RELU: return launch_nt1<VDSL_EPI_RELU>(a, b, C->ptr, c_dtype, pre, m, n, k, q->stream);
    default: return launch_nt1<VDSL_EPI_NONE>(a, b, C->ptr, c_dtype, pre, m, n, k, q->stream);
  }
}
