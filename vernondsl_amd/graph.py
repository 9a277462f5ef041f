"""Execution graph with reverse-mode autodiff, replayed as one hipGraph.

The reference has no execution graph or autodiff (it has no runtime at all); this module is the
front end the north star asks for: a program of tensor ops is built once, the autodiff pass
appends the backward ops, every tensor gets a static device buffer, and the whole step is
recorded on one queue and replayed as a single hipGraph (no host work or allocation per step).

    g = Graph()
    x = g.input("X", (2048, 4096), "bf16")
    w1 = g.param("W1", (4096, 4096), "bf16")         # [out][in]
    h = g.linear(x, w1, act="gelu")                  # bf16, GELU fused into the GEMM epilogue
    y = g.linear(h, g.param("W2", (4096, 4096), "bf16"), out_dtype="f32")
    loss = g.mse_loss(y, g.input("T", (2048, 4096), "f32"))
    grads = g.backward(loss)                         # {param name: gradient Value (f32)}
    exe = g.compile(dev)
    exe.write(q, "X", x_host) ...; step = exe.capture(q); step.launch(q)
    exe.write(q, "W1", w1_new); step.launch(q)       # re-packs W1 first, then replays

Backward rules (y = act(x W^T), W stored [out][in]):
    g    = dL/dy (+ its transpose g^T), bf16; for act = gelu / relu: g = gelu_bwd / relu_bwd(dL/dh, pre)
    dW   = g^T x        -> vdsl_op_gemm_bf16(A = g^T [out][B], B = x [B][in], trans_b = 0)
    dx   = g W          -> vdsl_op_gemm_bf16(A = g [B][out], B = W [out][in], trans_b = 0)
    MSE: loss and dL/dy = 2 (y - t) / n (bf16, plus transpose) from one fused op.
    y = a + b: dL/da = dL/db = dL/dy.
    A value read by several ops (a residual input, a weight tied across layers): dL/dv is the f32
    sum of the terms its readers give (an add op per extra term); fusions that would apply a term
    before the sum is complete (GELU' in the dL/dx GEMM, the loss in the last GEMM) are skipped
    for such values.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import _lib, kernels
from .rhi import Device, Queue, Tensor


@dataclass
class Value:
    name: str
    shape: tuple
    dtype: str
    kind: str = "activation"   # input | param | activation | grad | scratch
    producer: "Op | None" = None
    requires_grad: bool = False


@dataclass
class Op:
    kind: str
    inputs: list
    outputs: list
    attrs: dict = field(default_factory=dict)


class Graph:
    def __init__(self, prepare_transposes: bool = False, fuse_gelu_backward: bool = False,
                 pack_weights: bool = False, fuse_mse: bool = False, keep_y: bool = True,
                 store_gelu_deriv: bool = False, k_major_grads: bool = False):
        # prepare_transposes: backward() takes a param's transpose (the NT form's B of dL/dx) from a
        # prepare op instead of transposing the param inside every step's GEMM.
        # fuse_gelu_backward (needs prepare_transposes): GELU' is applied in the epilogue of the GEMM
        # that forms dL/dy of a GELU output (vdsl_op_gemm_bf16_gelu_bwd) instead of by a separate op.
        # Both off by default: measured on config 4 in one process, the step took 445.6 us as is,
        # 462 us with the transpose prepared (the transpose's 11.6 us gone, yet the back-to-back
        # GEMMs slower: they are power-bound and a memory-bound kernel between them lets the clock
        # recover) and 450 us with both (the fused GEMM 94 us against 100 us for GEMM + transpose +
        # GELU backward, the next forward GEMM 13 us slower).
        self.prepare_transposes = prepare_transposes
        self.fuse_gelu_backward = fuse_gelu_backward
        # pack_weights: linear ops on a param weight read a copy packed into MFMA fragment order
        # (vdsl_op_gemm_bf16_packed), made by a prepare op; same results bit for bit.
        self.pack_weights = pack_weights
        # fuse_mse: backward() merges an MSE loss with the packed, activation-free linear op that
        # produces its input (vdsl_op_gemm_bf16_mse_packed), so y never makes a round trip through
        # memory before the loss; keep_y: that op still stores y (the gradient does not need it).
        self.fuse_mse = fuse_mse
        self.keep_y = keep_y
        # store_gelu_deriv (with fuse_gelu_backward and packed weights): the forward GELU GEMM stores
        # GELU'(pre) instead of pre (VDSL_EPI_GELU_DERIV, sharing erfc with GELU), and the fused
        # backward GEMM multiplies by it (vdsl_op_gemm_bf16_mul_packed) instead of evaluating GELU'
        # after its main loop; the same products rounded the same way, bit for bit.
        self.store_gelu_deriv = store_gelu_deriv
        # k_major_grads: a weight-gradient GEMM dW = g^T x takes g as stored ([batch][out], trans_a,
        # read K-major by the GEMM) instead of g^T, and the transposed gradients that no op then
        # reads are elided: not allocated, not written (the epilogues that form g skip them).
        self.k_major_grads = k_major_grads
        self.elided: set = set()
        self._transposed: set = set()
        self.values: dict[str, Value] = {}
        self.ops: list[Op] = []
        # Ops that derive constant operands from params (weight packing): run by
        # Executable.prepare() after the params are written, never inside the replayed step.
        self.prepare_ops: list[Op] = []
        self._n = 0

    # ---- construction -------------------------------------------------------------------------
    def _value(self, name, shape, dtype, kind="activation", requires_grad=False) -> Value:
        if name in self.values:
            raise ValueError(f"duplicate tensor name {name!r}")
        v = Value(name, tuple(int(s) for s in shape), dtype, kind, None, requires_grad)
        self.values[name] = v
        return v

    def _fresh(self, base):
        self._n += 1
        return f"{base}#{self._n}"

    def _op(self, kind, inputs, outputs, **attrs) -> Op:
        op = Op(kind, list(inputs), list(outputs), attrs)
        for o in outputs:
            o.producer = op
        self.ops.append(op)
        return op

    def input(self, name, shape, dtype) -> Value:
        return self._value(name, shape, dtype, "input")

    def param(self, name, shape, dtype, requires_grad=True) -> Value:
        return self._value(name, shape, dtype, "param", requires_grad)

    def linear(self, x: Value, w: Value, act: str = "none", out_dtype: str | None = None, name=None) -> Value:
        """y = act(x W^T); x [B][in] bf16, W [out][in] bf16 (K-contiguous: the native MFMA layout)."""
        if x.dtype != "bf16" or w.dtype != "bf16":
            raise TypeError("linear takes bf16 activations and weights")
        if x.shape[1] != w.shape[1]:
            raise ValueError(f"linear: x {x.shape} and W {w.shape} disagree on the input width")
        if act not in ("none", "gelu", "relu"):
            raise ValueError(f"unknown activation {act!r}")
        out_dtype = out_dtype or ("bf16" if act != "none" else "f32")
        y = self._value(name or self._fresh("linear"), (x.shape[0], w.shape[0]), out_dtype,
                        requires_grad=x.requires_grad or w.requires_grad)
        pre = None
        if act != "none":
            pre = self._value(self._fresh("pre"), y.shape, "f32")  # kept for the backward pass
        packed = None
        if self.pack_weights and w.kind == "param" and w.shape[0] % 32 == 0 and w.shape[1] % 256 == 0:
            packed = self._prepared(w, "packed", w.shape, "pack_bf16")
        self._op("linear", [x, w], [y] + ([pre] if pre else []), act=act, pre=pre, packed=packed)
        return y

    def _prepared(self, w: Value, suffix: str, shape, kind: str) -> Value:
        """The value a prepare op of `kind` derives from param w (once per write of w, outside the
        replayed step); one per (w, kind)."""
        name = f"{w.name}.{suffix}"
        if name in self.values:
            return self.values[name]
        v = self._value(name, shape, w.dtype, "param")
        op = Op(kind, [w], [v])
        v.producer = op
        self.prepare_ops.append(op)
        return v

    def add(self, a: Value, b: Value, out_dtype: str | None = None, name=None) -> Value:
        """a + b elementwise (a residual sum): f32 or bf16 operands of one shape, one f32 addition,
        rounded to out_dtype (default f32 when either operand is f32, else bf16)."""
        if a.shape != b.shape:
            raise ValueError(f"add: shapes {a.shape} and {b.shape} differ")
        if a.dtype not in ("f32", "bf16") or b.dtype not in ("f32", "bf16"):
            raise TypeError("add takes f32 and bf16 tensors")
        out_dtype = out_dtype or ("f32" if "f32" in (a.dtype, b.dtype) else "bf16")
        if out_dtype not in ("f32", "bf16"):
            raise TypeError("add stores f32 or bf16")
        y = self._value(name or self._fresh("add"), a.shape, out_dtype, requires_grad=a.requires_grad or b.requires_grad)
        self._op("add", [a, b], [y])
        return y

    def mse_loss(self, y: Value, t: Value, name="loss") -> Value:
        if y.dtype != "f32" or t.dtype != "f32" or y.shape != t.shape:
            raise TypeError("mse_loss takes two f32 tensors of one shape")
        loss = self._value(name, (1,), "f32", requires_grad=y.requires_grad)
        self._op("mse", [y, t], [loss])
        return loss

    def quant_linear(self, x: Value, wq: Value, w_scale: Value, relu: bool, out_dtype="bf16", name=None,
                     packed: bool | None = None) -> Value:
        """y = relu?(dequant(q(x) wq^T)): per-row dynamic int8 activations, int8 weights [out][in]
        with per-output-channel f32 scales; int32 accumulation on MFMA.

        packed (default: whenever the shape allows it, out % 32 == 0 and in % 512 == 0): the
        step reads a copy of wq in MFMA fragment order, made by a prepare op (once per write of
        wq, outside the replayed step); same results bit for bit."""
        if wq.dtype != "i8" or w_scale.dtype != "f32":
            raise TypeError("quant_linear takes int8 weights and f32 scales")
        rows, k = x.shape
        n = wq.shape[0]
        if packed is None:
            packed = n % 32 == 0 and k % 512 == 0 and k > 0
        xq = self._value(self._fresh("xq"), (rows, k), "i8")
        xs = self._value(self._fresh("xscale"), (rows,), "f32")
        self._op("quantize", [x], [xq, xs])
        y = self._value(name or self._fresh("qlinear"), (rows, n), out_dtype)
        if packed:
            wp = self._value(self._fresh(f"{wq.name}.packed"), wq.shape, "i8", "param")
            op = Op("pack_w8a8", [wq], [wp])
            wp.producer = op
            self.prepare_ops.append(op)
            self._op("w8a8_packed", [xq, xs, wp, w_scale], [y], relu=bool(relu))
        else:
            self._op("w8a8", [xq, xs, wq, w_scale], [y], relu=bool(relu))
        return y

    # ---- autodiff --------------------------------------------------------------------------------
    def backward(self, loss: Value) -> dict:
        """Appends the backward ops of `loss` and returns {param name: f32 gradient Value}."""
        if loss.producer is None or loss.producer.kind != "mse":
            raise ValueError("backward() starts from an mse_loss value")
        fwd_ops = list(self.ops)
        uses: dict[str, int] = {}  # forward reads of each value: more than one means summed gradients
        for op in fwd_ops:
            for v in op.inputs:
                uses[v.name] = uses.get(v.name, 0) + 1
        # gradient of each activation: ("bf16", g, g_t) or ("f32", g)
        grad: dict[str, tuple] = {}
        y, _ = loss.producer.inputs
        dy = self._value(self._fresh("d_" + y.name), y.shape, "bf16", "grad")
        dy_t = self._value(self._fresh("dT_" + y.name), y.shape[::-1], "bf16", "grad")
        self._transposed.add(dy_t.name)
        part = self._value(self._fresh("mse_partials"), (max(1, kernels.mse_partials_count(*y.shape)),), "f32", "scratch")
        loss.producer.outputs += [dy, dy_t, part]  # the forward MSE op also emits dL/dy
        grad[y.name] = ("bf16", dy, dy_t)
        lin = y.producer
        if (self.fuse_mse and lin is not None and lin.kind == "linear" and lin.attrs["act"] == "none"
                and uses[y.name] == 1 and lin.attrs.get("packed") is not None and y.dtype == "f32"
                and y.shape[0] % 128 == 0 and y.shape[1] % 256 == 0):
            # the linear op and the loss become one op: the GEMM's epilogue forms the loss and dL/dy
            mse_op = loss.producer
            self.ops.remove(mse_op)
            lin.kind = "linear_mse"
            lin.inputs.append(mse_op.inputs[1])
            lin.outputs += [loss, dy, dy_t, part]
            for v in (loss, dy, dy_t, part):
                v.producer = lin
            if not self.keep_y:  # the fused op does not store y: nothing holds it
                self.elided.add(y.name)
        contrib: dict[str, list] = {}  # param name -> its gradient's terms, one per linear op reading it
        for op in reversed(fwd_ops):
            if op.kind == "mse":
                continue
            if op.kind not in ("linear", "linear_mse", "add"):
                raise NotImplementedError(f"no backward rule for {op.kind}")
            y = op.outputs[0]
            if y.name not in grad:
                continue
            if op.kind == "add":  # d(a + b) passes dL/dy to both operands
                for x in op.inputs:
                    if x.requires_grad or (x.producer is not None and x.kind == "activation" and _needs(x, self)):
                        self._accumulate(grad, x, grad[y.name])
                continue
            x, w = op.inputs[:2]
            g = grad[y.name]
            act = op.attrs["act"]
            if act == "gelu":
                if g[0] == "gelu_da":  # the GEMM that formed dL/dy already applied GELU'
                    gb, gt = g[1], g[2]
                else:
                    if g[0] != "f32":
                        g = self._to_f32(g[1])
                    da = self._value(self._fresh("d_pre"), y.shape, "bf16", "grad")
                    da_t = self._value(self._fresh("dT_pre"), y.shape[::-1], "bf16", "grad")
                    self._transposed.add(da_t.name)
                    self._op("gelu_bwd", [g[1], op.attrs["pre"]], [da, da_t])
                    gb, gt = da, da_t
            elif act == "none":
                if g[0] == "f32":
                    gb, gt = self._to_bf16_pair(g[1])
                else:
                    gb, gt = g[1], g[2]
            else:  # relu: dL/dpre = dL/dy where pre > 0
                if g[0] != "f32":
                    g = self._to_f32(g[1])
                da = self._value(self._fresh("d_pre"), y.shape, "bf16", "grad")
                da_t = self._value(self._fresh("dT_pre"), y.shape[::-1], "bf16", "grad")
                self._transposed.add(da_t.name)
                self._op("relu_bwd", [g[1], op.attrs["pre"]], [da, da_t])
                gb, gt = da, da_t
            if w.requires_grad:
                single = uses[w.name] == 1
                dw = self._value("grad_" + w.name if single else self._fresh("dterm_" + w.name), w.shape, "f32", "grad")
                # dW[out][in] = sum_b g[b][out] x[b][in]: A = g^T [out][B] (K = B contiguous), B = x [B][in];
                # with k_major_grads A is g as stored ([B][out] = [K][M], trans_a)
                if self.k_major_grads:
                    self._op("gemm", [gb, x], [dw], trans_a=True, trans_b=False, epi=_lib.EPI_NONE)
                else:
                    self._op("gemm", [gt, x], [dw], trans_a=False, trans_b=False, epi=_lib.EPI_NONE)
                contrib.setdefault(w.name, []).append(dw)
            if x.requires_grad or (x.producer is not None and x.kind == "activation" and _needs(x, self)):
                # dx[B][in] = sum_o g[b][o] W[o][in]: A = g [B][out], B = W stored [out][in] = [K][N].
                # A param's transpose W^T [in][out] (the NT form's B) is made once by a prepare op
                # instead of by the GEMM on every step.
                wt = self._param_transpose(w) if self.prepare_transposes and w.kind == "param" else None
                xp = x.producer
                if (self.fuse_gelu_backward and wt is not None and xp is not None and xp.kind == "linear"
                        and xp.attrs["act"] == "gelu" and uses[x.name] == 1):
                    # x = GELU(pre): the GEMM's epilogue applies GELU'(pre) and emits dL/dpre (bf16,
                    # plus its transpose) without writing dL/dx
                    da = self._value(self._fresh("d_pre"), x.shape, "bf16", "grad")
                    da_t = self._value(self._fresh("dT_pre"), x.shape[::-1], "bf16", "grad")
                    self._transposed.add(da_t.name)
                    packed = self.pack_weights and wt.shape[0] % 32 == 0 and wt.shape[1] % 256 == 0
                    if packed:  # W^T packed into MFMA fragment order (a second prepare op)
                        wt = self._prepared(wt, "packed", wt.shape, "pack_bf16")
                    if packed and self.store_gelu_deriv and xp.attrs.get("packed") is not None:
                        # the forward op keeps GELU'(pre) in place of pre, which nothing else reads
                        pre = xp.attrs["pre"]
                        dg = self._value(self._fresh("dgelu"), pre.shape, "f32")
                        xp.outputs[xp.outputs.index(pre)] = dg
                        dg.producer = xp
                        del self.values[pre.name]
                        xp.attrs["pre"], xp.attrs["dgelu"] = None, dg
                        self._op("gemm_mul_bwd", [gb, wt, dg], [da, da_t])
                    else:
                        self._op("gemm_gelu_bwd", [gb, wt, xp.attrs["pre"]], [da, da_t], packed=packed)
                    grad[x.name] = ("gelu_da", da, da_t)
                else:
                    dx = self._value(self._fresh("d_" + x.name), x.shape, "f32", "grad")
                    if wt is not None:
                        self._op("gemm", [gb, wt], [dx], trans_a=False, trans_b=True, epi=_lib.EPI_NONE)
                    else:
                        self._op("gemm", [gb, w], [dx], trans_a=False, trans_b=False, epi=_lib.EPI_NONE)
                    self._accumulate(grad, x, ("f32", dx))
        param_grads = {}
        for name, terms in contrib.items():
            # a param read by several linear ops (tied weights): the sum of its terms, in the order
            # backward formed them (the last forward use first), named grad_<param> at the end
            acc = terms[0]
            for k, t in enumerate(terms[1:], 2):
                last = k == len(terms)
                s = self._value("grad_" + name if last else self._fresh("dsum_" + name), acc.shape, "f32", "grad")
                self._op("add", [acc, t], [s])
                acc = s
            param_grads[name] = acc
        if self.k_major_grads:
            self._elide_unread_transposes()
        return param_grads

    def _accumulate(self, grad: dict, x: Value, g: tuple):
        """Adds the gradient term g to dL/dx: the first term is kept as it is; a second one (x read
        by several ops) makes dL/dx their f32 sum, formed by an add op."""
        prev = grad.get(x.name)
        if prev is None:
            grad[x.name] = g
            return
        if "gelu_da" in (prev[0], g[0]):
            raise AssertionError("a GELU backward was fused for a value with several readers")
        a = prev[1] if prev[0] == "f32" else self._to_f32(prev[1])
        b = g[1] if g[0] == "f32" else self._to_f32(g[1])
        s = self._value(self._fresh("dsum_" + x.name), x.shape, "f32", "grad")
        self._op("add", [a, b], [s])
        grad[x.name] = ("f32", s)

    def _elide_unread_transposes(self):
        """Transposed gradients no op reads: a transpose op that makes one is dropped; one emitted
        beside its untransposed form by a loss or GEMM epilogue (which accepts no transposed output)
        is marked elided, so the executable neither allocates nor writes it."""
        read = {v.name for op in self.ops + self.prepare_ops for v in op.inputs}
        dead = {n for n in self._transposed if n not in read}
        for op in list(self.ops):
            if op.kind == "transpose" and op.outputs[0].name in dead:
                self.ops.remove(op)
                del self.values[op.outputs[0].name]
        self.elided |= {n for n in dead if n in self.values}

    def _param_transpose(self, w: Value) -> Value:
        """W^T of a param, made by a prepare op (once per write of W, outside the replayed step)."""
        return self._prepared(w, "T", w.shape[::-1], "transpose")

    def _to_f32(self, v: Value) -> Value:
        o = self._value(self._fresh(v.name + "_f32"), v.shape, "f32", "grad")
        self._op("cast", [v], [o])
        return o

    def _to_bf16_pair(self, v: Value):
        b = self._value(self._fresh(v.name + "_bf16"), v.shape, "bf16", "grad")
        bt = self._value(self._fresh(v.name + "_bf16T"), v.shape[::-1], "bf16", "grad")
        self._transposed.add(bt.name)
        self._op("cast", [v], [b])
        self._op("transpose", [b], [bt])
        return b, bt

    # ---- compile ---------------------------------------------------------------------------------
    def compile(self, dev: Device) -> "Executable":
        return Executable(self, dev)

    def host_outputs(self) -> set:
        """Values an op produces and no op (step or prepare) reads: results for the host only.  Their
        buffers are bound as VDSL_BIND_OUTPUT, which lets a GEMM store an f32 result with streaming
        (non-temporal) stores instead of leaving it dirty in the caches for the next kernels."""
        read = {v.name for op in self.ops + self.prepare_ops for v in op.inputs}
        return {v.name for op in self.ops for v in op.outputs if v.kind != "scratch"} - read - self.elided


def _needs(x: Value, g: Graph) -> bool:
    """An activation needs a gradient if some parameter upstream of it requires one."""
    seen, stack = set(), [x]
    while stack:
        v = stack.pop()
        if v.name in seen:
            continue
        seen.add(v.name)
        if v.kind == "param" and v.requires_grad:
            return True
        if v.producer is not None:
            stack.extend(v.producer.inputs)
    return False


class Executable:
    """Static buffers for every value, the op sequence bound to them, and hipGraph capture."""

    def __init__(self, g: Graph, dev: Device):
        self.graph = g
        self.dev = dev
        self.t: dict[str, Tensor] = {}
        self.workspace = None
        self._stale: set[str] = {v.name for op in g.prepare_ops for v in op.inputs}
        ws = 0
        for op in g.ops:
            if op.kind == "gemm":
                a, b = op.inputs
                M, K = (a.shape[1], a.shape[0]) if op.attrs["trans_a"] else a.shape
                N = b.shape[0] if op.attrs["trans_b"] else b.shape[1]
                ws = max(ws, kernels.gemm_bf16_workspace_bytes(op.attrs["trans_a"], op.attrs["trans_b"], M, N, K))
            if op.kind == "w8a8":
                xq, _, wq, _ = op.inputs
                ws = max(ws, kernels.gemm_w8a8_workspace_bytes(xq.shape[0], wq.shape[0], xq.shape[1]))
            if op.kind == "w8a8_packed":
                xq, _, wp, _ = op.inputs
                ws = max(ws, kernels.gemm_w8a8_packed_workspace_bytes(xq.shape[0], wp.shape[0], xq.shape[1]))
        outs = g.host_outputs()
        try:
            for v in g.values.values():
                if v.name in g.elided:
                    self.t[v.name] = None  # never written: the ops that could emit it are told to skip it
                    continue
                bind = _lib.BIND_OUTPUT if v.name in outs else _lib.BIND_STORAGE_BUFFER
                self.t[v.name] = Tensor(dev, v.shape, v.dtype, bind)
            # One workspace shared by all ops: they run in order on one queue.
            self.workspace = Tensor(dev, (max(ws, 4),), "i8") if ws else None
        except BaseException:
            self.free()  # an allocation failed: release what was allocated before re-raising
            raise

    def write(self, q: Queue, name: str, host):
        if self.t.get(name, 0) is None:
            raise KeyError(f"{name} is elided from this graph (no op stores it: a transposed gradient nothing reads, "
                           "see Graph.k_major_grads, or y of a fused loss built with keep_y=False)")
        self.t[name].buffer.write(q, host)
        if any(v.name == name for op in self.graph.prepare_ops for v in op.inputs):
            self._stale.add(name)

    def prepare(self, q: Queue):
        """Runs the prepare ops (weight packing, param transposes) whose params were written since
        they last ran.  run(), capture() and every Step.launch() call it first, so no step reads
        packed or transposed weights older than the params they derive from."""
        T = self.t
        for op in self.graph.prepare_ops:  # in order: an op may read what an earlier one made
            if op.inputs[0].name not in self._stale:
                continue
            self._stale.update(v.name for v in op.outputs)
            if op.kind == "pack_w8a8":
                kernels.pack_w8a8_weights(q, T[op.inputs[0].name], T[op.outputs[0].name])
            elif op.kind == "transpose":
                kernels.transpose(q, T[op.inputs[0].name], T[op.outputs[0].name])
            elif op.kind == "pack_bf16":
                kernels.pack_bf16_weights(q, T[op.inputs[0].name], T[op.outputs[0].name])
            else:
                raise NotImplementedError(op.kind)
        self._stale.clear()

    def read(self, q: Queue, name: str):
        if self.t.get(name, 0) is None:
            raise KeyError(f"{name} is elided from this graph (no op stores it: a transposed gradient nothing reads, "
                           "see Graph.k_major_grads, or y of a fused loss built with keep_y=False)")
        return self.t[name].numpy(q)

    def run(self, q: Queue, events=None):
        """Enqueues every op of the graph, in order, on q (after any pending prepare ops, unless q
        is recording a capture).  events: optional rhi.Events, one per op, each recorded on q right
        after its op (per-op timing of the step as it runs)."""
        if self._stale and not q.capturing:
            self.prepare(q)
        if events is not None and len(events) != len(self.graph.ops):
            raise ValueError(f"{len(events)} events for {len(self.graph.ops)} ops")
        for i, op in enumerate(self.graph.ops):
            self._run_op(q, op)
            if events is not None:
                events[i].record(q)

    def op_label(self, op: Op) -> str:
        """A short description of one op: its kind, form and extents (M x N x K for GEMMs)."""
        ins, outs = op.inputs, op.outputs
        if op.kind == "linear":
            (M, K), N = ins[0].shape, ins[1].shape[0]
            form = "packed" if op.attrs.get("packed") is not None else "row-major"
            return f"linear {op.attrs['act']} ({form} weights, {outs[0].dtype} out) {M}x{N}x{K}"
        if op.kind == "linear_mse":
            (M, K), N = ins[0].shape, ins[1].shape[0]
            return f"linear + MSE loss and dL/dy (packed weights) {M}x{N}x{K}"
        if op.kind == "gemm":
            a, b = ins
            M, K = (a.shape[1], a.shape[0]) if op.attrs["trans_a"] else a.shape
            N = b.shape[0] if op.attrs["trans_b"] else b.shape[1]
            return f"gemm {'T' if op.attrs['trans_a'] else 'N'}{'T' if op.attrs['trans_b'] else 'N'} {M}x{N}x{K}"
        if op.kind == "gemm_gelu_bwd":
            (M, K), N = ins[0].shape, ins[1].shape[0]
            return f"gemm + GELU backward ({'packed' if op.attrs.get('packed') else 'row-major'} B) {M}x{N}x{K}"
        if op.kind == "gemm_mul_bwd":
            (M, K), N = ins[0].shape, ins[1].shape[0]
            return f"gemm x stored GELU' (packed B) {M}x{N}x{K}"
        if op.kind in ("w8a8", "w8a8_packed"):
            (M, K), N = ins[0].shape, ins[2].shape[0]
            return f"{op.kind} {'relu' if op.attrs['relu'] else 'no relu'} {M}x{N}x{K}"
        return f"{op.kind} {'x'.join(map(str, ins[0].shape))}"

    def op_flops(self, op: Op) -> int:
        """2 M N K for a GEMM op (multiply-adds of its main loop), 0 otherwise."""
        ins = op.inputs
        if op.kind in ("linear", "gemm_gelu_bwd", "gemm_mul_bwd", "linear_mse"):
            return 2 * ins[0].shape[0] * ins[0].shape[1] * ins[1].shape[0]
        if op.kind == "gemm":
            a, b = ins
            M, K = (a.shape[1], a.shape[0]) if op.attrs["trans_a"] else a.shape
            N = b.shape[0] if op.attrs["trans_b"] else b.shape[1]
            return 2 * M * N * K
        if op.kind in ("w8a8", "w8a8_packed"):
            return 2 * ins[0].shape[0] * ins[0].shape[1] * ins[2].shape[0]
        return 0

    def _run_op(self, q: Queue, op: Op):
        T = self.t
        ins = [T[v.name] for v in op.inputs]
        outs = [T[v.name] for v in op.outputs]
        if op.kind == "linear":
            pre = T[op.attrs["pre"].name] if op.attrs["pre"] is not None else None
            epi = {"none": _lib.EPI_NONE, "gelu": _lib.EPI_GELU, "relu": _lib.EPI_RELU}[op.attrs["act"]]
            if op.attrs.get("dgelu") is not None:  # GELU'(pre) stored in place of pre
                epi, pre = _lib.EPI_GELU_DERIV, T[op.attrs["dgelu"].name]
            if op.attrs.get("packed") is not None:
                kernels.gemm_bf16_packed(q, ins[0], T[op.attrs["packed"].name], outs[0], epi, pre)
            else:
                kernels.gemm_bf16(q, ins[0], ins[1], outs[0], trans_a=False, trans_b=True, epilogue=epi,
                                  pre_act=pre)
        elif op.kind == "gemm":
            kernels.gemm_bf16(q, ins[0], ins[1], outs[0], op.attrs["trans_a"], op.attrs["trans_b"], op.attrs["epi"],
                              None, self.workspace)
        elif op.kind == "linear_mse":
            y, loss, dy, dy_t, part = outs
            kernels.gemm_bf16_mse_packed(q, ins[0], T[op.attrs["packed"].name], ins[2], y if self.graph.keep_y else None,
                                         loss, dy, dy_t, part)
        elif op.kind == "mse":
            loss = outs[0]
            if len(outs) == 4:
                kernels.mse_fwd_bwd(q, ins[0], ins[1], loss, outs[1], outs[2], outs[3])
            else:
                raise RuntimeError("mse without backward: call Graph.backward() or use the loss op's fused form")
        elif op.kind == "gelu_bwd":
            kernels.gelu_bwd(q, ins[0], ins[1], outs[0], outs[1])
        elif op.kind == "relu_bwd":
            kernels.gelu_bwd(q, ins[0], ins[1], outs[0], outs[1], act="relu")
        elif op.kind == "add":
            kernels.add(q, ins[0], ins[1], outs[0])
        elif op.kind == "gemm_gelu_bwd":
            kernels.gemm_bf16_gelu_bwd(q, ins[0], ins[1], ins[2], outs[0], outs[1], op.attrs.get("packed", False))
        elif op.kind == "gemm_mul_bwd":
            kernels.gemm_bf16_mul_packed(q, ins[0], ins[1], ins[2], outs[0], outs[1])
        elif op.kind == "cast":
            kernels.cast(q, ins[0], outs[0])
        elif op.kind == "transpose":
            kernels.transpose(q, ins[0], outs[0])
        elif op.kind == "quantize":
            kernels.quantize_rows_i8(q, ins[0], outs[0], outs[1])
        elif op.kind == "w8a8":
            kernels.gemm_w8a8(q, ins[0], ins[1], ins[2], ins[3], outs[0], op.attrs["relu"], None, self.workspace)
        elif op.kind == "w8a8_packed":
            kernels.gemm_w8a8_packed(q, ins[0], ins[1], ins[2], ins[3], outs[0], op.attrs["relu"], None,
                                     self.workspace)
        else:
            raise NotImplementedError(op.kind)

    def capture(self, q: Queue) -> "Step":
        """Records one run() into a hipGraph and returns it as a Step (.launch(q), .destroy()).
        Pending prepare ops run first, eagerly, outside the recording."""
        if self._stale:
            self.prepare(q)
        with q.capture() as rec:
            self.run(q)
        return Step(self, rec.graph)

    def free(self):
        for t in self.t.values():
            if t is not None:
                t.free()
        self.t = {}
        if self.workspace is not None:
            self.workspace.free()
            self.workspace = None


class Step:
    """One captured step of an Executable.  The recording reads the prepared operands (packed
    weights, param transposes) from their static buffers, so launch() first re-runs, eagerly on
    the same queue and outside the recording, the prepare ops of any param written with
    Executable.write() since the last launch; the replay then reads the new weights."""

    def __init__(self, exe: Executable, g):
        self.exe = exe
        self.graph = g

    @property
    def handle(self):
        return self.graph.handle

    def launch(self, q: Queue):
        if self.exe._stale:
            self.exe.prepare(q)
        self.graph.launch(q)

    def destroy(self):
        self.graph.destroy()


# ---- the two workload graphs ------------------------------------------------------------------------
def mlp_train_graph(batch=2048, d_in=4096, hidden=4096, d_out=4096, prepare_transposes=True,
                    fuse_gelu_backward=True, pack_weights=True, fuse_mse=True, keep_y=True, store_gelu_deriv=True,
                    k_major_grads=True):
    """Config 4: X -> GELU(X W1^T) -> (.) W2^T -> MSE(., T), with backward for W1 and W2.

    The defaults are the fastest form measured on MI355X (one process, graph replays, same
    gradients bit for bit as the plain graph with none of the options)."""
    g = Graph(prepare_transposes, fuse_gelu_backward, pack_weights, fuse_mse, keep_y, store_gelu_deriv, k_major_grads)
    x = g.input("X", (batch, d_in), "bf16")
    w1 = g.param("W1", (hidden, d_in), "bf16")
    w2 = g.param("W2", (d_out, hidden), "bf16")
    t = g.input("T", (batch, d_out), "f32")
    h = g.linear(x, w1, act="gelu", name="H")
    y = g.linear(h, w2, out_dtype="f32", name="Y")
    loss = g.mse_loss(y, t)
    grads = g.backward(loss)
    return g, grads


def w8a8_infer_graph(batch=512, widths=(8192, 8192, 8192, 8192, 1024)):
    """Config 5: int8 MLP, ReLU between layers, bf16 activations."""
    g = Graph()
    h = g.input("X", (batch, widths[0]), "bf16")
    for li in range(len(widths) - 1):
        wq = g.param(f"W{li}", (widths[li + 1], widths[li]), "i8", requires_grad=False)
        ws = g.param(f"S{li}", (widths[li + 1],), "f32", requires_grad=False)
        last = li == len(widths) - 2
        h = g.quant_linear(h, wq, ws, relu=not last, name="Y" if last else f"H{li}")
    return g
