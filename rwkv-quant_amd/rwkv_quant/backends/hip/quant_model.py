"""RWKV-7 x070 inference on a `.rwkvq` checkpoint through the HIP kernels.

Same interface as the reference Metal model
(reference: rwkv_quant/backends/metal/quant_model.py:838-990):

    model = QuantRWKV7(ckpt)                 # QuantizedCheckpoint
    states = model.init_state(B)
    logits, states = model.forward_stateful(idx[B, T], states,
                                            last_only=False, tail_only=0)
    logits, states = model.step(idx, states)  # decode: HIP-graph replay
    hidden, states = model.forward_hidden(idx, states)
    logits = model(idx)

State per layer: (wkv [B, H, N, N] fp32, time-mix shift [B, 1, D] or None,
channel-mix shift [B, 1, D] or None), None meaning a zero shift on the
first call (reference: quant_model.py:902-908).  Tensors live on the GPU.

Execution per layer (every numeric step is a librwkvq_hip kernel):
  shift_lerp(ln1, 6 lerps) -> fused r/k/v GEMV (one launch) ->
  LoRA down (4 branches, one launch) -> LoRA up (one launch) ->
  wkv_prep -> wkv7_scan -> wkv_tail -> o_proj GEMV (+= residual) ->
  shift_lerp(ln2, 1 lerp) -> key GEMV (relu^2) -> value GEMV (+= residual)
Decode (T = 1) runs LoRA up + prep + one recurrence step + tail as one
launch per (sequence, head).  On a world checkpoint the decode LoRA reads
the file's codes (asym gw64 / per-row int8, exact weights) instead of the
fp16 copies the prefill GEMMs use.
Prefill (B*T >= GEMM_MIN_BATCH_NB) runs the projections on the MFMA GEMM
kernel (dequantization fused into the operand load, epilogue fused, the
r/k/v triple in one launch) and the LoRA products as fp16 GEMMs.

Runtime switches (module attributes, as the reference's FUSE flags):
  FUSE        fuse r/k/v into one GEMV launch at decode
  FUSE_DECODE decode (T = 1): the LoRA up products folded into the WKV
              step (one launch fewer per layer)
  USE_GRAPH   replay decode steps from a captured HIP graph
  LORA_FROM_CODES  decode LoRA from the file's codes (world checkpoints)
  PERSISTENT_DECODE  batch-1 decode: every layer in one persistent launch
              (rwkvq_decode_mk; five grid-barrier phases per layer) where
              the model's shape and formats allow it
"""
import ctypes
from collections import OrderedDict

import torch

from . import _lib
from .quant_linear import (GEMM_MIN_BATCH_NB, GwQuantLinear,
                           GwQuantLinearFused, QuantLinearV2, SymQuantLinear,
                           SymQuantLinearFused, make_linear, spqr_csr)
from .repack import lora_codes_ok, lora_down_device, lora_up_device

FUSE = True
FUSE_DECODE = True
USE_GRAPH = True
LORA_KERNEL_MAX_N = 8          # rows handled by the grouped LoRA kernel
DOWN_SEG_MIN_N = 3             # decode rows from which the LoRA down
                               # products take the segmented MFMA GEMV
WKV_CHUNK_MIN_T = 32           # sequence length from which the WKV scan
                               # runs in 16-step chunks (operators + a
                               # sequential pass on the matrix cores)
WKV_CHUNK_OPS = 6400           # operator floats per (sequence, head, chunk)
WKV_PREP_FUSED = True          # chunked prefill: per-channel prep inside the
                               # chunk-operator kernel
X16_PREFILL = True             # prefill GEMM inputs written as fp16 in the
                               # GEMM's pair order by their producers
LORA_GEMV_ROWS = 32            # decode-batch rows per LoRA-down GEMV launch
LORA_FROM_CODES = True         # decode LoRA (world checkpoints) read from
                               # the file's codes instead of fp16 copies
                               # (checked at run time, like FUSE_DECODE)
LORA_Q_MAX_NC = 16384          # rows x width the code-based down kernel
                               # stages in LDS (64 KiB of fp32 x)
PERSISTENT_DECODE = True       # batch-1 decode layers in one launch
MAX_SEQ_GRAPHS = 8             # captured forward_stateful graphs kept (LRU);
                               # each owns its logits and two state sets

_LORA = ("w1", "w2", "a1", "a2", "v1", "v2", "g1", "g2")


def _stream():
    return _lib.stream_handle()


def dense_param(qt, device):
    """QuantizedTensor -> exact float32 device tensor in stored orientation.
    Quantized tensors are expanded by the bit-exact dequant kernels."""
    shape = tuple(qt.shape)
    if qt.bits >= 16:
        return qt.dense.to(device=device, dtype=torch.float32).reshape(shape)
    rows = shape[0]
    cols = 1
    for s in shape[1:]:
        cols *= s
    out = torch.empty((rows, cols), dtype=torch.float32, device=device)
    if qt.gw_mode == "asym":
        codes = qt.codes.to(device).view(torch.uint8).contiguous()
        sc = qt.gw_scale.to(device).float().contiguous()
        mn = qt.gw_min.to(device).float().contiguous()
        _lib.call("rwkvq_dequant_asym_f32", _lib.ptr(codes), _lib.ptr(sc),
                  _lib.ptr(mn), qt.gw_gs, rows, cols, _lib.ptr(out), cols,
                  _stream())
    elif qt.gw_mode == "" and qt.codes is not None and qt.bits <= 8:
        codes = qt.codes.to(device).view(torch.int8).reshape(rows, cols) \
            .contiguous()
        sc = qt.scale.to(device).view(torch.int16).reshape(rows).contiguous()
        _lib.call("rwkvq_dequant_rtn8_f32", _lib.ptr(codes), _lib.ptr(sc),
                  rows, cols, _lib.ptr(out), cols, _stream())
        if qt.outlier_indices is not None and qt.outlier_indices.numel():
            ptr, col, val = spqr_csr(qt, device)
            _lib.call("rwkvq_spqr_scatter", _lib.ptr(ptr), _lib.ptr(col),
                      _lib.ptr(val), rows, _lib.ptr(out), cols, _stream())
    elif qt.gw_mode in ("sb6", "sym") or qt.gw_mode == "":
        lin = make_linear(qt, device)
        lin._dequant_into(out)
    else:
        raise NotImplementedError(f"dense_param: {qt.gw_mode!r}")
    return out.reshape(shape)


class EmbTable:
    """Token embedding: row gather straight from the packed table."""

    def __init__(self, qt, device):
        self.vocab, self.dim = qt.shape
        self.device = device
        self.dense = None
        if qt.bits >= 16:
            self.dense = qt.dense.to(device=device, dtype=torch.float32)
            return
        self.lin = make_linear(qt, device)
        if isinstance(self.lin, GwQuantLinear):
            self.kind, self.bits = 0, self.lin.bits
            self.args = (self.lin.nib, self.lin.hb, self.lin.rec, None)
        elif isinstance(self.lin, SymQuantLinear):
            self.kind, self.bits = 1, self.lin.bits
            self.args = (self.lin.codes, self.lin.hb, self.lin.qs, self.lin.d)
        elif isinstance(self.lin, QuantLinearV2):
            if self.lin.has_outliers:
                raise NotImplementedError("rtn emb with outliers")
            self.kind, self.bits = 2, 8
            self.args = (self.lin.codes, None, None, self.lin.scale)
        else:
            raise NotImplementedError(type(self.lin))

    def gather_into(self, idx, out):
        """idx int64 [n] on device -> out [n, D] fp32."""
        if self.dense is not None:
            torch.index_select(self.dense, 0, idx, out=out)
            return out
        q, hb, a0, a1 = self.args
        _lib.call("rwkvq_gather_rows_f32", self.kind, self.bits, _lib.ptr(q),
                  _lib.ptr(hb), _lib.ptr(a0), _lib.ptr(a1), self.vocab,
                  self.dim, _lib.ptr(idx), idx.numel(), _lib.ptr(out),
                  _stream())
        return out

    def gather_ln_into(self, idx, w, b, eps, out):
        """out [n, D] = LayerNorm(emb[idx]) with (w, b, eps): one launch for
        a packed table (bit-exact with gather_into + rwkvq_layer_norm)."""
        if self.dense is not None:
            self.gather_into(idx, out)
            _lib.call("rwkvq_layer_norm", _lib.ptr(out), _lib.ptr(w),
                      _lib.ptr(b), _lib.ptr(out), idx.numel(), self.dim, eps,
                      _stream())
            return out
        q, hb, a0, a1 = self.args
        _lib.call("rwkvq_gather_ln_f32", self.kind, self.bits, _lib.ptr(q),
                  _lib.ptr(hb), _lib.ptr(a0), _lib.ptr(a1), self.vocab,
                  self.dim, _lib.ptr(idx), idx.numel(), _lib.ptr(w),
                  _lib.ptr(b), eps, _lib.ptr(out), _stream())
        return out


class _Work:
    """Activation buffers for N = B*T rows (reused across layers)."""

    def __init__(self, N, C, ffn, ranks, device):
        f = dict(dtype=torch.float32, device=device)
        self.N = N
        self.x = torch.empty(N, C, **f)          # residual stream
        self.xs = torch.empty(N, 6, C, **f)      # r, k, v, w, a, g lerps
        self.rkv = torch.empty(N, 3, C, **f)
        self.h = {b: torch.empty(N, r, **f) for b, r in ranks.items()}
        # prefill LoRA: the down outputs of all branches, each padded to a
        # multiple of 128
        rp = sum(-(-r // 128) * 128 for r in ranks.values())
        self.h_cat = torch.empty(N, rp, **f) if N > 8 else None
        self.yl = {b: torch.empty(N, C, **f) for b in ranks}
        self.w = torch.empty(N, C, **f)
        self.kp = torch.empty(N, C, **f)
        self.vp = torch.empty(N, C, **f)
        self.aa = torch.empty(N, C, **f)
        self.bb = torch.empty(N, C, **f)
        self.y = torch.empty(N, C, **f)
        self.o = torch.empty(N, C, **f)
        self.v_first = torch.empty(N, C, **f)
        self.xk = torch.empty(N, C, **f)
        self.hk = torch.empty(N, ffn, **f)
        self.xo = torch.empty(N, C, **f)
        if N >= GEMM_MIN_BATCH_NB:
            # prefill GEMM inputs as fp16, each in its GEMM's pair order
            h = dict(dtype=torch.float16, device=device)
            self.xs16 = torch.empty(N, 6, C, **h)
            self.o16 = torch.empty(N, C, **h)
            self.xk16 = torch.empty(N, C, **h)
            self.hk16 = torch.empty(N, ffn, **h)
            self.h16 = torch.empty(N, rp, **h)
        self.device = device
        self.wkv_ops = None

    def wkv_ops_buffer(self, H):
        """Chunk-operator workspace of the chunked WKV scan, sized once for
        the largest need of any split N = B * T (T >= WKV_CHUNK_MIN_T), so
        it is never reallocated: HIP graphs captured for one (B, T) keep
        pointing at it while other shapes of the same N run (allocated by
        the warm-up run that precedes any capture)."""
        if self.wkv_ops is None:
            self.wkv_ops = torch.empty(wkv_ops_floats(self.N, H),
                                       dtype=torch.float32,
                                       device=self.device)
        return self.wkv_ops


def wkv_chunk_slots(B, T):
    """Chunks per head of the chunked scan: ceil(T / 16) rounded up to a
    multiple of 3 (the scan applies three chunks per step)."""
    return B * (-(-(-(-T // 16)) // 3) * 3)


def wkv_ops_floats(N, H):
    """Operator floats of the chunked scan for the worst split of N rows
    into B sequences of T >= WKV_CHUNK_MIN_T tokens."""
    slots = max([wkv_chunk_slots(B, N // B) for B in range(1, N + 1)
                 if N % B == 0 and N // B >= WKV_CHUNK_MIN_T] or [0])
    return max(1, slots * H * WKV_CHUNK_OPS)


def _lora_codes(g, branches, C, head_size, device):
    """Device layouts of the decode LoRA factors read straight from the
    file's codes (world checkpoint: down stored [C, rank], up [rank, C]);
    None when a factor's format or shape does not allow it."""
    if head_size != 64 or C not in (2048, 2560, 4096):
        return None
    on = lambda a: None if a is None else torch.from_numpy(a).to(device)
    cpu = lambda t: None if t is None else t.detach().cpu().numpy()
    out = {}
    for b in branches:
        dq, uq = g(b + "1"), g(b + "2")
        if not (lora_codes_ok(dq, 1, lambda c: c % 16 == 0)
                and dq.shape[0] == C
                and lora_codes_ok(uq, 16, lambda c: c == C)
                and uq.shape[0] == dq.shape[1]):
            return None
        lays = []
        for qt, fn in ((dq, lora_down_device), (uq, lora_up_device)):
            if qt.gw_mode == "asym":
                lay = fn(cpu(qt.codes), tuple(qt.shape), scale=cpu(qt.gw_scale),
                         mn=cpu(qt.gw_min))
            else:
                lay = fn(cpu(qt.codes), tuple(qt.shape),
                         row_scale=cpu(qt.scale))
            lays.append({k: on(v) for k, v in lay.items()})
        out[b] = (dq.shape[1], lays[0], lays[1])
    return out


class QuantTMix:
    def __init__(self, tensors, prefix, naming, layer_id, n_head, head_size,
                 device):
        self.H, self.S, self.layer_id = n_head, head_size, layer_id
        g = lambda s: tensors[prefix + s]
        dev = device
        if naming == "world":
            names = dict(x=["x_r", "x_k", "x_v", "x_w", "x_a", "x_g"],
                         r="receptance.weight", k="key.weight",
                         v="value.weight", o="output.weight",
                         w0="w0", a0="a0", v0="v0")
            pre = "att."

            def lora(nm, up):
                t = dense_param(g(pre + nm), dev)
                return t.t().contiguous()        # stored [in, out]
        else:
            names = dict(x=["x_r", "x_k", "x_v", "x_w", "x_a", "x_g"],
                         r="r_proj.weight", k="k_proj.weight",
                         v="v_proj.weight", o="o_proj.weight",
                         w0="w_lora_B.bias", a0="a_lora_B.bias",
                         v0="v_lora_B.bias")
            pre = "tmix."
            custom = {"w1": "w_lora_A.weight", "w2": "w_lora_B.weight",
                      "a1": "a_lora_A.weight", "a2": "a_lora_B.weight",
                      "v1": "v_lora_A.weight", "v2": "v_lora_B.weight",
                      "g1": "g_lora_A.weight", "g2": "g_lora_B.weight"}

            def lora(nm, up):
                return dense_param(g(pre + custom[nm]), dev)
        vec = lambda s: dense_param(g(pre + s), dev).reshape(-1).contiguous()
        # lerp coefficients in kernel order r, k, v, w, a, g
        self.coef = torch.stack([vec(s) for s in names["x"]]).contiguous()
        C = self.coef.shape[1]
        self.C = C
        self.r_proj = make_linear(g(pre + names["r"]), dev)
        self.k_proj = make_linear(g(pre + names["k"]), dev)
        self.v_proj = make_linear(g(pre + names["v"]), dev)
        self.o_proj = make_linear(g(pre + names["o"]), dev)
        self.w0 = vec(names["w0"])
        self.a0 = vec(names["a0"])
        self.v0 = vec(names["v0"]) if layer_id > 0 else None
        self.k_k, self.k_a, self.r_k = vec("k_k"), vec("k_a"), vec("r_k")
        self.ln_x_w, self.ln_x_b = vec("ln_x.weight"), vec("ln_x.bias")
        # LoRA: A [r, C] (down), B [C, r] (up), fp16 on device
        self.lora = {}
        for b in ("w", "a", "v", "g"):
            if b == "v" and layer_id == 0:
                continue
            A = lora(b + "1", False).to(torch.float16).contiguous()
            Bm = lora(b + "2", True).to(torch.float16).contiguous()
            self.lora[b] = (A, Bm)
        # the down factors stacked in lerp-slot order (v, w, a, g) in one
        # buffer (the per-branch A are views of it): one segmented launch
        # runs all down products of a decode batch
        self.down_order = [b for b in ("v", "w", "a", "g") if b in self.lora]
        A_cat = torch.cat([self.lora[b][0] for b in self.down_order]).contiguous()
        off = 0
        for b in self.down_order:
            r = self.lora[b][0].shape[0]
            self.lora[b] = (A_cat[off:off + r], self.lora[b][1])
            off += r
        self.down_cat = A_cat
        self.down_seg_ok = A_cat.shape[1] % 128 == 0 and all(
            self.lora[b][0].shape[0] % 16 == 0 for b in self.down_order)
        self.rkv_fused = None
        lins = [self.r_proj, self.k_proj, self.v_proj]
        if all(isinstance(l, GwQuantLinear) for l in lins) and \
                len({(l.in_features, l.out_features, l.bits)
                     for l in lins}) == 1:
            self.rkv_fused = GwQuantLinearFused(lins)
        elif all(isinstance(l, SymQuantLinear) for l in lins) and \
                all(lins[0].can_fuse_with(l) for l in lins):
            self.rkv_fused = SymQuantLinearFused(lins)

        # decode LoRA straight from the file's codes (world checkpoints)
        self.lora_q = None
        if naming == "world":
            self.lora_q = _lora_codes(lambda nm: g(pre + nm), list(self.lora),
                                      C, head_size, dev)
        # decode fusion (LoRA up into the WKV step) needs ranks the fused
        # WKV kernel tiles
        self.decode_fusable = (
            all(A.shape[0] % 8 == 0 for A, _ in self.lora.values())
            and sum(A.shape[0] for A, _ in self.lora.values()) <= 1024)

    # order of the lerp slots in work.xs
    SLOT = {"r": 0, "k": 1, "v": 2, "w": 3, "a": 4, "g": 5}
    EPI_DOWN = {"w": _lib.EPI_TANH, "a": _lib.EPI_STORE, "v": _lib.EPI_STORE,
                "g": _lib.EPI_SIGMOID}

    def run_lora(self, wk, x16_order=None):
        """x16_order (prefill): the lerp outputs are the fp16 wk.xs16 in
        that pair order; the down outputs go to wk.h16 as fp16."""
        N, C = wk.N, self.C
        branches = list(self.lora)
        if N <= LORA_KERNEL_MAX_N:
            self.run_lora_down(wk)
            W = [self.lora[b][1] for b in branches]
            X = [wk.h[b] for b in branches]
            self._grouped(W, X, [wk.h[b].shape[1] for b in branches],
                          [wk.yl[b] for b in branches],
                          [_lib.EPI_STORE] * len(branches), N)
            return
        if x16_order is None and N < GEMM_MIN_BATCH_NB:
            self._run_lora_batch(wk)
            return
        # prefill: the MFMA GEMM over the dense fp16 factors; one launch for
        # the down products of all branches (their lerp slots v, w, a, g are
        # adjacent in wk.xs), one per up product
        x16 = x16_order is not None
        order, rps, A_cat, B_pad, modes = self._prefill_mats(
            x16_order if x16 else _lib.ORDER_PAIRS)
        xs_flat = (wk.xs16 if x16 else wk.xs).view(N, 6 * C)
        hbuf = wk.h16 if x16 else wk.h_cat
        s0 = self.SLOT[order[0]]
        nseg, tot = len(order), sum(rps)
        flags = (_lib.X_F16 | _lib.Y_F16
                 | (_lib.ORDER_PAIRS << _lib.Y_ORDER_SHIFT)) if x16 else 0
        _lib.call("rwkvq_gemm_f16_seg", _lib.ptr(A_cat), nseg,
                  (ctypes.c_int * nseg)(*rps), C,
                  _lib.ptr(xs_flat[:, s0 * C:]), 6 * C, _lib.ptr(hbuf), N,
                  modes, flags, _stream())
        # the down GEMM wrote rows of `tot` values, branch j from column
        # sum(rps[:j]) on
        self._run_ups(wk, x16, order, rps, B_pad)

    def _run_lora_batch(self, wk):
        """Decode batches of 9..127 rows: the down products as the
        segmented matrix-core GEMV in 32-row launches (the padded stacked
        factors; a GEMM would have a handful of output tiles here), into
        per-branch padded buffers carved from wk.h_cat, then the up products
        in one grouped launch."""
        N, C = wk.N, self.C
        order, rps, A_cat, B_pad, modes = self._prefill_mats()
        nseg = len(order)
        hp = [wk.h_cat.view(-1)[N * sum(rps[:j]):N * sum(rps[:j + 1])]
              .view(N, rps[j]) for j in range(nseg)]
        xs_flat = wk.xs.view(N, 6 * C)
        x0 = xs_flat[:, self.SLOT[order[0]] * C:]
        rows = (ctypes.c_int * nseg)(*rps)
        for n0 in range(0, N, LORA_GEMV_ROWS):
            n = min(LORA_GEMV_ROWS, N - n0)
            ys = (ctypes.c_void_p * nseg)(*[h[n0:].data_ptr() for h in hp])
            _lib.call("rwkvq_gemv_f16_seg", _lib.ptr(A_cat), nseg, rows, C,
                      _lib.ptr(x0[n0:]), 6 * C, ys, n, modes, _stream())
        P = ctypes.c_void_p
        _lib.call("rwkvq_gemm_f16_grouped", nseg,
                  (P * nseg)(*[B_pad[b].data_ptr() for b in order]),
                  (ctypes.c_int * nseg)(*[C] * nseg),
                  (ctypes.c_int * nseg)(*rps),
                  (P * nseg)(*[h.data_ptr() for h in hp]),
                  (ctypes.c_long * nseg)(*rps),
                  (P * nseg)(*[wk.yl[b].data_ptr() for b in order]),
                  N, 0, 0, _stream())

    def run_rkv_lora_x16(self, wk, x_order):
        """Prefill with fp16 lerp outputs (pair order x_order): the r/k/v
        projection and the LoRA down products in one launch (the down
        tiles run on the CUs the r/k/v tiles leave free), then the ups."""
        N, C = wk.N, self.C
        rf = self.rkv_fused
        kind, lead = rf._cat._kargs()
        if kind == "sb6":
            k, (p0, p1, p2, bits), p3 = 0, lead, None
        elif kind == "sym":
            k, (p0, p1, p2, p3, bits) = 1, lead
        else:
            k, (p0, p3), p1, p2, bits = 2, lead, None, None, 8
        order, rps, A_cat, B_pad, modes = self._prefill_mats(x_order)
        xs_flat = wk.xs16.view(N, 6 * C)
        nseg = len(order)
        _lib.call("rwkvq_gemm_dual_f16seg", k, bits, p0, p1, p2, p3,
                  rf.out_features, rf.in_features, rf.out_per,
                  _lib.ptr(wk.xs16), 6 * C, _lib.ptr(wk.rkv), _lib.X_F16,
                  _lib.ptr(A_cat), nseg, (ctypes.c_int * nseg)(*rps),
                  _lib.ptr(xs_flat[:, self.SLOT[order[0]] * C:]), 6 * C,
                  _lib.ptr(wk.h16), modes,
                  _lib.X_F16 | _lib.Y_F16
                  | (_lib.ORDER_PAIRS << _lib.Y_ORDER_SHIFT), N, _stream())
        self._run_ups(wk, True, order, rps, B_pad)

    def _run_ups(self, wk, x16, order, rps, B_pad):
        """The up products of all branches in one launch, from the down
        outputs (wk.h16 fp16 or wk.h_cat fp32, branch j from column
        sum(rps[:j]) on, rows of sum(rps) values)."""
        N, C = wk.N, self.C
        nseg, tot = len(order), sum(rps)
        hbuf = wk.h16 if x16 else wk.h_cat
        hc = hbuf.view(-1)[:N * tot].view(N, tot)
        # branch j reads its rps[j] columns
        offs = [sum(rps[:j]) for j in range(nseg)]
        P = ctypes.c_void_p
        _lib.call("rwkvq_gemm_f16_grouped", nseg,
                  (P * nseg)(*[B_pad[b].data_ptr() for b in order]),
                  (ctypes.c_int * nseg)(*[C] * nseg),
                  (ctypes.c_int * nseg)(*rps),
                  (P * nseg)(*[hc[:, o:].data_ptr() for o in offs]),
                  (ctypes.c_long * nseg)(*[tot] * nseg),
                  (P * nseg)(*[wk.yl[b].data_ptr() for b in order]),
                  N, 0, _lib.X_F16 if x16 else 0, _stream())

    def _prefill_mats(self, x_order=_lib.ORDER_PAIRS):
        """Prefill LoRA factors padded for the GEMM tiles (built on first
        use): down factors stacked in lerp-slot order (v, w, a, g), each
        padded with zero rows to a multiple of 128 (rps), their columns in
        pair order x_order (that of the fp16 lerp outputs they read: the
        GEMM pairs halves 2i, 2i+1, so permuting W's columns like x's keeps
        the product); up factors padded with zero columns to the same
        width.  Padded outputs multiply zero weights."""
        cache = self.__dict__.setdefault("_pmats_by_order", {})
        if x_order not in cache:
            order, rps, A_cat, B_pad, modes = self._prefill_mats_base()
            if x_order != _lib.ORDER_PAIRS:
                C = self.C
                idx = torch.as_tensor(pair_cols(x_order), device=A_cat.device)
                idx = (torch.arange(0, C, 32, device=A_cat.device)[:, None]
                       + idx[None]).reshape(-1)
                A_cat = A_cat[:, idx].contiguous()
            cache[x_order] = (order, rps, A_cat, B_pad, modes)
        return cache[x_order]

    def _prefill_mats_base(self):
        if getattr(self, "_pmats", None) is None:
            order = [b for b in ("v", "w", "a", "g") if b in self.lora]
            C = self.C
            rps = [-(-self.lora[b][0].shape[0] // 128) * 128 for b in order]
            A0 = self.lora[order[0]][0]
            A_cat = torch.zeros(sum(rps), C, dtype=torch.float16,
                                device=A0.device)
            B_pad = {}
            off = 0
            for j, b in enumerate(order):
                A, Bm = self.lora[b]
                r = A.shape[0]
                A_cat[off:off + r] = A
                Bp = torch.zeros(C, rps[j], dtype=torch.float16,
                                 device=A0.device)
                Bp[:, :r] = Bm
                B_pad[b] = Bp
                off += rps[j]
            modes = 0
            for j, b in enumerate(order):
                modes |= self.EPI_DOWN[b] << (4 * j)
            self._pmats = (order, rps, A_cat, B_pad, modes)
        return self._pmats

    def run_lora_down(self, wk):
        """The down products only (decode with the up products folded into
        the WKV step): one launch, results (after tanh / sigmoid) in
        wk.h[b].  Three or more rows: the segmented matrix-core GEMV over
        the stacked factors; fewer: the grouped lane-dot kernel."""
        N, C = wk.N, self.C
        xs_flat = wk.xs.view(N, 6 * C)
        if (LORA_FROM_CODES and self.lora_q is not None
                and N * C <= LORA_Q_MAX_NC):
            br = list(self.lora_q)
            n = len(br)
            P = ctypes.c_void_p
            lay = [self.lora_q[b][1] for b in br]
            pa = lambda key: (P * n)(*[None if l[key] is None
                                       else l[key].data_ptr() for l in lay])
            ia = lambda v: (ctypes.c_int * n)(*v)
            _lib.call("rwkvq_lora_down_q", n, pa("q"), pa("s"), pa("m"),
                      pa("sc"),
                      (P * n)(*[xs_flat[:, self.SLOT[b] * C:].data_ptr()
                                for b in br]),
                      ia([6 * C] * n), (P * n)(*[wk.h[b].data_ptr() for b in br]),
                      ia([wk.h[b].shape[1] for b in br]),
                      ia([self.lora_q[b][0] for b in br]),
                      ia([self.EPI_DOWN[b] for b in br]), C, N, _stream())
            return
        if N >= DOWN_SEG_MIN_N and self.down_seg_ok and N <= 16:
            order = self.down_order
            rows = (ctypes.c_int * len(order))(
                *[self.lora[b][0].shape[0] for b in order])
            ys = (ctypes.c_void_p * len(order))(
                *[wk.h[b].data_ptr() for b in order])
            modes = 0
            for j, b in enumerate(order):
                modes |= self.EPI_DOWN[b] << (4 * j)
            _lib.call("rwkvq_gemv_f16_seg", _lib.ptr(self.down_cat),
                      len(order), rows, C,
                      _lib.ptr(xs_flat[:, self.SLOT[order[0]] * C:]), 6 * C,
                      ys, N, modes, _stream())
            return
        br = list(self.lora)
        self._grouped([self.lora[b][0] for b in br],
                      [xs_flat[:, self.SLOT[b] * C:] for b in br],
                      [6 * C] * len(br), [wk.h[b] for b in br],
                      [self.EPI_DOWN[b] for b in br], N)

    def wkv_decode_lora(self, wk, wkv_in, wkv_out, layer0, B, H, S):
        """Decode WKV step with the LoRA up products folded in."""
        order = ("w", "a", "v", "g")
        have = [b in self.lora for b in order]
        if LORA_FROM_CODES and self.lora_q is not None:
            P = ctypes.c_void_p
            ups = [self.lora_q[b][2] if h else None
                   for b, h in zip(order, have)]
            pa = lambda key: (P * 4)(*[None if u is None or u[key] is None
                                       else u[key].data_ptr() for u in ups])
            _lib.call("rwkvq_wkv7_decode_lora_q", _lib.ptr(wk.rkv),
                      (P * 4)(*[wk.h[b].data_ptr() if h else None
                                for b, h in zip(order, have)]),
                      pa("q"), pa("s"), pa("m"), pa("sc"),
                      (ctypes.c_int * 4)(*[self.lora_q[b][0] if h else 0
                                           for b, h in zip(order, have)]),
                      _lib.ptr(self.w0), _lib.ptr(self.a0), _lib.ptr(self.v0),
                      _lib.ptr(self.k_k), _lib.ptr(self.k_a),
                      _lib.ptr(self.r_k), _lib.ptr(self.ln_x_w),
                      _lib.ptr(self.ln_x_b), _lib.ptr(wk.v_first), layer0,
                      _lib.ptr(wkv_in), _lib.ptr(wkv_out), _lib.ptr(wk.o), B,
                      H, S, _stream())
            return
        hp = (ctypes.c_void_p * 4)(*[wk.h[b].data_ptr() if h else None
                                     for b, h in zip(order, have)])
        bp = (ctypes.c_void_p * 4)(*[self.lora[b][1].data_ptr() if h
                                     else None for b, h in zip(order, have)])
        rk = (ctypes.c_int * 4)(*[self.lora[b][0].shape[0] if h else 0
                                  for b, h in zip(order, have)])
        _lib.call("rwkvq_wkv7_decode_lora", _lib.ptr(wk.rkv), hp, bp, rk,
                  _lib.ptr(self.w0), _lib.ptr(self.a0), _lib.ptr(self.v0),
                  _lib.ptr(self.k_k), _lib.ptr(self.k_a), _lib.ptr(self.r_k),
                  _lib.ptr(self.ln_x_w), _lib.ptr(self.ln_x_b),
                  _lib.ptr(wk.v_first), layer0, _lib.ptr(wkv_in),
                  _lib.ptr(wkv_out), _lib.ptr(wk.o), B, H, S, _stream())

    @staticmethod
    def _grouped(W, X, x_ld, Y, epi, N):
        """One rwkvq_lora_gemv launch over the branches (host arrays of
        pointers and sizes; the kernel receives them by value)."""
        n = len(W)
        vp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in W])
        xp = (ctypes.c_void_p * n)(*[x.data_ptr() for x in X])
        yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in Y])
        ia = lambda v: (ctypes.c_int * n)(*v)
        _lib.call("rwkvq_lora_gemv", n, vp, xp, ia(x_ld), yp,
                  ia([y.shape[1] for y in Y]), ia([w.shape[0] for w in W]),
                  ia([w.shape[1] for w in W]), ia(epi), N, _stream())


class QuantCMix:
    def __init__(self, tensors, prefix, naming, device):
        pre = "cmix." if naming == "custom" else "ffn."
        g = lambda s: tensors[prefix + pre + s]
        self.x_k = dense_param(g("x_k"), device).reshape(1, -1).contiguous()
        self.key = make_linear(g("key.weight"), device)
        self.value = make_linear(g("value.weight"), device)


class QuantBlock:
    def __init__(self, tensors, prefix, naming, layer_id, n_head, head_size,
                 device):
        vec = lambda s: dense_param(tensors[prefix + s], device).reshape(-1) \
            .contiguous()
        self.ln1_w, self.ln1_b = vec("ln1.weight"), vec("ln1.bias")
        self.ln2_w, self.ln2_b = vec("ln2.weight"), vec("ln2.bias")
        self.tmix = QuantTMix(tensors, prefix, naming, layer_id, n_head,
                              head_size, device)
        self.cmix = QuantCMix(tensors, prefix, naming, device)


def pair_cols(order):
    """Source column of each fp16 position of a 32-column group in pair
    order `order` (RWKVQ_ORDER_*): halves 2i, 2i+1 hold (c0(i), c1(i))."""
    cols = []
    for i in range(16):
        if order == _lib.ORDER_SB6:
            cols += [i, i + 16]
        elif order == _lib.ORDER_SYM6:
            c0 = i if i < 8 else i + 8
            cols += [c0, c0 + 8]
        else:
            cols += [2 * i, 2 * i + 1]
    return cols


def _x16_orders(blk):
    """Pair orders of the fp16 inputs of the block's prefill GEMMs (r/k/v,
    output, channel-mix key, value), or None where a matrix has no fp16
    input path (dense fallback, rtn outliers, shapes off the MFMA tiles)."""
    tm, cm = blk.tmix, blk.cmix
    rf = tm.rkv_fused
    if not FUSE or rf is None or not rf._cat.gemm_ok(rf.out_per):
        return None
    lins = (rf, tm.o_proj, cm.key, cm.value)
    orders = [getattr(l, "x16_order", None) for l in lins]
    if any(o is None for o in orders) or not all(
            l.gemm_ok() for l in lins[1:]):
        return None
    return orders


def _apply(lin, x2, y, mode, n=None, x_ld=0):
    """y <- epi(x2 @ W^T): GEMV kernel for small N, MFMA GEMM for prefill
    (both with the epilogue fused)."""
    return lin.apply_into(x2, y, mode=mode, n=n, x_ld=x_ld)


class QuantRWKV7:
    def __init__(self, ckpt, device="cuda"):
        _lib.load()
        self.device = torch.device(device)
        self.naming = ckpt.naming
        self.n_layer = ckpt.n_layer
        self.n_embd = ckpt.n_embd
        self.head_size = ckpt.head_size
        self.n_head = ckpt.n_embd // ckpt.head_size
        self.vocab_size = ckpt.vocab_size
        if self.head_size != 64:
            raise NotImplementedError("HIP WKV kernels are built for head 64")
        t = ckpt.tensors
        dev = self.device
        self.emb = EmbTable(t["emb.weight"], dev)
        self.head = make_linear(t["head.weight"], dev)
        vec = lambda k: dense_param(t[k], dev).reshape(-1).contiguous()
        if self.naming == "custom":
            self.ln0_w, self.ln0_b = vec("ln0.weight"), vec("ln0.bias")
        else:
            self.ln0_w, self.ln0_b = vec("blocks.0.ln0.weight"), \
                vec("blocks.0.ln0.bias")
        self.ln_out_w, self.ln_out_b = vec("ln_out.weight"), vec("ln_out.bias")
        self.blocks = [QuantBlock(t, f"blocks.{i}.", self.naming, i,
                                  self.n_head, self.head_size, dev)
                       for i in range(self.n_layer)]
        b0 = self.blocks[-1]
        self.ffn = b0.cmix.key.out_features
        self.ranks = {b: A.shape[0] for b, (A, _) in
                      self.blocks[-1].tmix.lora.items()}
        self._work = {}
        self._graphs = {}              # decode step graphs by batch size
        self._seq_graphs = OrderedDict()   # forward graphs by shape (LRU)
        self._mk = None                # persistent decode (built on first use)
        torch.cuda.synchronize(dev)

    # ------------------------------------------------------------ state
    def init_state(self, batch_size=1):
        H, S = self.n_head, self.head_size
        return [(torch.zeros(batch_size, H, S, S, device=self.device), None,
                 None) for _ in range(self.n_layer)]

    def _work_for(self, N):
        if N not in self._work:
            self._work[N] = _Work(N, self.n_embd, self.ffn, self.ranks,
                                  self.device)
        return self._work[N]

    def _persistent(self, B, T):
        """The persistent decode kernel's host object when this step
        (B sequences, T tokens) runs on it, else None."""
        if not (PERSISTENT_DECODE and B == 1 and T == 1):
            return None
        if self._mk is None:
            from .decode_mk import PersistentDecode
            self._mk = PersistentDecode(self)
        return self._mk if self._mk.ok else None

    # ---------------------------------------------------------- forward
    def _idx(self, idx):
        idx = torch.as_tensor(idx)
        if idx.dim() == 1:
            idx = idx[None]
        if not idx.is_cuda:
            if idx.numel() and (int(idx.min()) < 0
                                or int(idx.max()) >= self.vocab_size):
                raise ValueError("token id out of range")
        return idx.to(device=self.device, dtype=torch.int64)

    def _body(self, idx, states, wk, out_states):
        """All layers for idx [B, T] (device int64); writes the new state
        tensors into out_states (preallocated) and leaves ln_out(x) in
        wk.xo."""
        B, T = idx.shape
        N, C, H = B * T, self.n_embd, self.n_head
        st = _stream()
        x = wk.x
        self.emb.gather_ln_into(idx.reshape(-1), self.ln0_w, self.ln0_b, 1e-5,
                                x)
        mk = self._persistent(B, T)
        if mk is not None:
            mk.run(states, out_states, wk, st)
            _lib.call("rwkvq_layer_norm", _lib.ptr(x),
                      _lib.ptr(self.ln_out_w), _lib.ptr(self.ln_out_b),
                      _lib.ptr(wk.xo), N, C, 1e-5, st)
            return
        x16 = (X16_PREFILL and T > 1 and N >= GEMM_MIN_BATCH_NB
               and N > LORA_KERNEL_MAX_N)
        for li, (blk, state) in enumerate(zip(self.blocks, states)):
            tm, cm = blk.tmix, blk.cmix
            wkv_in, tshift, cshift = state
            wkv_out, tshift_out, cshift_out = out_states[li]
            layer0 = 1 if li == 0 else 0
            orders = _x16_orders(blk) if x16 else None
            if orders is not None:
                self._layer_x16(blk, orders, x, tshift, cshift, wkv_in,
                                wkv_out, tshift_out, cshift_out, layer0, wk,
                                B, T)
                continue
            _lib.call("rwkvq_shift_lerp", _lib.ptr(x), _lib.ptr(blk.ln1_w),
                      _lib.ptr(blk.ln1_b), _lib.ptr(tshift),
                      _lib.ptr(tm.coef), 6, _lib.ptr(wk.xs),
                      _lib.ptr(tshift_out), B, T, C, st)
            if FUSE and tm.rkv_fused is not None and (
                    N < GEMM_MIN_BATCH_NB
                    or tm.rkv_fused._cat.gemm_ok(tm.rkv_fused.out_per)):
                tm.rkv_fused.apply_into(wk.xs, wk.rkv, N, 6 * C)
            else:
                xs_flat = wk.xs.view(N, 6 * C)
                rkv_flat = wk.rkv.view(N, 3 * C)
                for j, lin in enumerate((tm.r_proj, tm.k_proj, tm.v_proj)):
                    tmp = torch.empty(N, C, device=self.device)
                    _apply(lin, xs_flat[:, j * C:], tmp, _lib.EPI_STORE,
                           n=N, x_ld=6 * C)
                    rkv_flat[:, j * C:(j + 1) * C].copy_(tmp)
            fused = (T == 1 and FUSE_DECODE and tm.decode_fusable
                     and N <= LORA_KERNEL_MAX_N)
            if fused:
                # LoRA up folded into the WKV step: 2 launches for LoRA + WKV
                tm.run_lora_down(wk)
                tm.wkv_decode_lora(wk, wkv_in, wkv_out, layer0, B, H,
                                   self.head_size)
            elif T == 1:
                tm.run_lora(wk)
                _lib.call("rwkvq_wkv7_decode", _lib.ptr(wk.rkv),
                          _lib.ptr(wk.yl["w"]), _lib.ptr(wk.yl["a"]),
                          None if layer0 else _lib.ptr(wk.yl["v"]),
                          _lib.ptr(wk.yl["g"]), _lib.ptr(tm.w0),
                          _lib.ptr(tm.a0), _lib.ptr(tm.v0), _lib.ptr(tm.k_k),
                          _lib.ptr(tm.k_a), _lib.ptr(tm.r_k),
                          _lib.ptr(tm.ln_x_w), _lib.ptr(tm.ln_x_b),
                          _lib.ptr(wk.v_first), layer0, _lib.ptr(wkv_in),
                          _lib.ptr(wkv_out), _lib.ptr(wk.o), B, H,
                          self.head_size, st)
            else:
                tm.run_lora(wk)
                self._wkv_seq(tm, wk, wkv_in, wkv_out, layer0, B, T, st)
            _apply(tm.o_proj, wk.o, x, _lib.EPI_ADD)
            _lib.call("rwkvq_shift_lerp", _lib.ptr(x), _lib.ptr(blk.ln2_w),
                      _lib.ptr(blk.ln2_b), _lib.ptr(cshift),
                      _lib.ptr(cm.x_k), 1, _lib.ptr(wk.xk),
                      _lib.ptr(cshift_out), B, T, C, st)
            _apply(cm.key, wk.xk, wk.hk, _lib.EPI_RELU2)
            _apply(cm.value, wk.hk, x, _lib.EPI_ADD)
        _lib.call("rwkvq_layer_norm", _lib.ptr(x), _lib.ptr(self.ln_out_w),
                  _lib.ptr(self.ln_out_b), _lib.ptr(wk.xo), N, C, 1e-5, st)

    def _layer_x16(self, blk, orders, x, tshift, cshift, wkv_in, wkv_out,
                   tshift_out, cshift_out, layer0, wk, B, T):
        """One prefill layer with every GEMM input fp16, written by its
        producer in the GEMM's pair order: the lerp kernel (r/k/v + LoRA
        down, channel-mix key), the time-mix tail (output projection), the
        key GEMM's epilogue (value)."""
        tm, cm = blk.tmix, blk.cmix
        N, C = B * T, self.n_embd
        st = _stream()
        o_r, o_o, o_k, o_v = orders
        _lib.call("rwkvq_shift_lerp_f16", _lib.ptr(x), _lib.ptr(blk.ln1_w),
                  _lib.ptr(blk.ln1_b), _lib.ptr(tshift), _lib.ptr(tm.coef), 6,
                  _lib.ptr(wk.xs16), o_r, _lib.ptr(tshift_out), B, T, C, st)
        tm.run_rkv_lora_x16(wk, o_r)
        self._wkv_seq(tm, wk, wkv_in, wkv_out, layer0, B, T, st, o16=o_o)
        tm.o_proj.apply_into(wk.o16, x, mode=_lib.EPI_ADD | _lib.X_F16, n=N)
        _lib.call("rwkvq_shift_lerp_f16", _lib.ptr(x), _lib.ptr(blk.ln2_w),
                  _lib.ptr(blk.ln2_b), _lib.ptr(cshift), _lib.ptr(cm.x_k), 1,
                  _lib.ptr(wk.xk16), o_k, _lib.ptr(cshift_out), B, T, C, st)
        cm.key.apply_into(wk.xk16, wk.hk16, n=N,
                          mode=(_lib.EPI_RELU2 | _lib.X_F16 | _lib.Y_F16
                                | (o_v << _lib.Y_ORDER_SHIFT)))
        cm.value.apply_into(wk.hk16, x, mode=_lib.EPI_ADD | _lib.X_F16, n=N)

    def _wkv_seq(self, tm, wk, wkv_in, wkv_out, layer0, B, T, st, o16=None):
        """T > 1: per-channel inputs, the scan (step by step, or from
        WKV_CHUNK_MIN_T on in 16-step chunks), tail."""
        N, C, H = B * T, self.n_embd, self.n_head
        if T >= WKV_CHUNK_MIN_T and WKV_PREP_FUSED:
            # prep folded into the chunk operators: two launches
            ops = wk.wkv_ops_buffer(H)
            _lib.call("rwkvq_wkv7_prefill_chunked", _lib.ptr(wk.rkv),
                      _lib.ptr(wk.yl["w"]), _lib.ptr(wk.yl["a"]),
                      None if layer0 else _lib.ptr(wk.yl["v"]),
                      _lib.ptr(tm.w0), _lib.ptr(tm.a0), _lib.ptr(tm.v0),
                      _lib.ptr(tm.k_k), _lib.ptr(tm.k_a),
                      _lib.ptr(wk.v_first), layer0, _lib.ptr(wk.kp),
                      _lib.ptr(wk.vp), _lib.ptr(wkv_in), _lib.ptr(wkv_out),
                      _lib.ptr(wk.y), B, T, H, self.head_size, _lib.ptr(ops),
                      ops.numel(), st)
            self._wkv_tail(tm, wk, N, C, st, o16)
            return
        _lib.call("rwkvq_wkv_prep", _lib.ptr(wk.rkv), _lib.ptr(wk.yl["w"]),
                  _lib.ptr(wk.yl["a"]),
                  None if layer0 else _lib.ptr(wk.yl["v"]), _lib.ptr(tm.w0),
                  _lib.ptr(tm.a0), _lib.ptr(tm.v0), _lib.ptr(tm.k_k),
                  _lib.ptr(tm.k_a), _lib.ptr(wk.v_first), layer0,
                  _lib.ptr(wk.w), _lib.ptr(wk.kp), _lib.ptr(wk.vp),
                  _lib.ptr(wk.aa), _lib.ptr(wk.bb), N, C, self.head_size, st)
        if T >= WKV_CHUNK_MIN_T:
            ops = wk.wkv_ops_buffer(H)
            _lib.call("rwkvq_wkv7_scan_chunked", _lib.ptr(wk.rkv), 3 * C,
                      _lib.ptr(wk.w), _lib.ptr(wk.kp), _lib.ptr(wk.vp),
                      _lib.ptr(wk.aa), _lib.ptr(wk.bb), C, _lib.ptr(wkv_in),
                      _lib.ptr(wkv_out), _lib.ptr(wk.y), C, B, T, H,
                      self.head_size, _lib.ptr(ops), ops.numel(), st)
        else:
            _lib.call("rwkvq_wkv7_scan", _lib.ptr(wk.rkv), 3 * C,
                      _lib.ptr(wk.w), _lib.ptr(wk.kp), _lib.ptr(wk.vp),
                      _lib.ptr(wk.aa), _lib.ptr(wk.bb), C, _lib.ptr(wkv_in),
                      _lib.ptr(wkv_out), _lib.ptr(wk.y), C, B, T, H,
                      self.head_size, st)
        self._wkv_tail(tm, wk, N, C, st, o16)

    def _wkv_tail(self, tm, wk, N, C, st, o16):
        """Group norm + bonus + gate into wk.o (fp32) or wk.o16 (fp16 in the
        output projection's pair order o16)."""
        if o16 is not None:                 # fp16 in the o GEMM's order
            _lib.call("rwkvq_wkv_tail_f16", _lib.ptr(wk.y), _lib.ptr(wk.rkv),
                      _lib.ptr(wk.kp), _lib.ptr(wk.vp), _lib.ptr(wk.yl["g"]),
                      _lib.ptr(tm.r_k), _lib.ptr(tm.ln_x_w),
                      _lib.ptr(tm.ln_x_b), _lib.ptr(wk.o16), o16, N, C,
                      self.head_size, st)
            return
        _lib.call("rwkvq_wkv_tail", _lib.ptr(wk.y), _lib.ptr(wk.rkv),
                  _lib.ptr(wk.kp), _lib.ptr(wk.vp), _lib.ptr(wk.yl["g"]),
                  _lib.ptr(tm.r_k), _lib.ptr(tm.ln_x_w), _lib.ptr(tm.ln_x_b),
                  _lib.ptr(wk.o), N, C, self.head_size, st)

    def _new_states(self, B):
        H, S, C = self.n_head, self.head_size, self.n_embd
        dev = self.device
        return [(torch.empty(B, H, S, S, device=dev),
                 torch.empty(B, 1, C, device=dev),
                 torch.empty(B, 1, C, device=dev))
                for _ in range(self.n_layer)]

    def forward_hidden(self, idx, states):
        """Hidden state after ln_out, before the head: [B, T, D]."""
        idx = self._idx(idx)
        B, T = idx.shape
        wk = self._work_for(B * T)
        out = self._new_states(B)
        self._body(idx, states, wk, out)
        return wk.xo.reshape(B, T, -1).clone(), out

    def forward_stateful(self, idx, states, last_only=False, tail_only=0):
        """idx [B, T] -> (logits [B, T', V], new_states).  With USE_GRAPH a
        HIP graph is captured once per (B, T, last_only, tail_only) and
        replayed (the analogue of the reference's compiled step, which
        traces once per shape: reference quant_model.py:910-942)."""
        idx = self._idx(idx)
        B, T = idx.shape
        if USE_GRAPH and T > 1:
            return self._replay_seq(idx, states, last_only, tail_only)
        out = self._new_states(B)
        logits = self._forward_into(idx, states, out, last_only, tail_only)
        return logits.reshape(B, -1, self.vocab_size), out

    def _forward_into(self, idx, states, out, last_only, tail_only,
                      logits=None):
        B, T = idx.shape
        wk = self._work_for(B * T)
        self._body(idx, states, wk, out)
        xo = wk.xo.reshape(B, T, -1)
        if last_only and T > 1:
            xo = xo[:, -1:]
        elif tail_only and T > tail_only:
            xo = xo[:, -tail_only:]
        xo = xo.reshape(-1, self.n_embd).contiguous()
        if logits is None:
            logits = torch.empty(xo.shape[0], self.vocab_size,
                                 device=self.device)
        _apply(self.head, xo, logits, _lib.EPI_STORE)
        return logits

    def _replay_seq(self, idx, states, last_only, tail_only):
        B, T = idx.shape
        key = (B, T, bool(last_only), int(tail_only))
        g = self._seq_graphs.get(key)
        if g is None:
            g = self._capture_seq(*key)
            self._seq_graphs[key] = g
            while len(self._seq_graphs) > MAX_SEQ_GRAPHS:
                self._seq_graphs.popitem(last=False)
        else:
            self._seq_graphs.move_to_end(key)
        g["idx"].copy_(idx)
        self._load_states(g["in"], states)
        g["graph"].replay()
        new = [(s.clone(), t.clone(), c.clone()) for s, t, c in g["out"]]
        return g["logits"].clone().reshape(B, -1, self.vocab_size), new

    @staticmethod
    def _load_states(dst, states):
        for (si, ti, ci), (wi, tsi, csi) in zip(dst, states):
            si.copy_(wi)
            if tsi is None:
                ti.zero_()
            else:
                ti.copy_(tsi)
            if csi is None:
                ci.zero_()
            else:
                ci.copy_(csi)

    def _capture_seq(self, B, T, last_only, tail_only):
        dev = self.device
        idx = torch.zeros(B, T, dtype=torch.int64, device=dev)
        st_in, st_out = self._new_states(B), self._new_states(B)
        for s in st_in:
            for t in s:
                t.zero_()
        rows = B if (last_only and T > 1) else (
            B * tail_only if (tail_only and T > tail_only) else B * T)
        logits = torch.empty(rows, self.vocab_size, device=dev)

        def run():
            self._forward_into(idx, st_in, st_out, last_only, tail_only,
                               logits)

        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            run()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run()
        torch.cuda.synchronize(dev)
        return {"graph": graph, "idx": idx, "in": st_in, "out": st_out,
                "logits": logits}

    def __call__(self, idx):
        idx = self._idx(idx)
        return self.forward_stateful(idx, self.init_state(idx.shape[0]))[0]

    # ------------------------------------------------- graph-replay decode
    def step(self, idx, states):
        """Decode step (T = 1 per sequence).  With USE_GRAPH the whole step
        is captured once per batch size into a HIP graph with static
        buffers and replayed; states are copied into / out of the graph's
        buffers (device-to-device)."""
        idx = self._idx(idx)
        B, T = idx.shape
        if not USE_GRAPH or T != 1:
            return self.forward_stateful(idx, states)
        g = self._graphs.get(B)
        if g is None:
            g = self._capture(B)
            self._graphs[B] = g
        g["idx"].copy_(idx)
        g["next"] = 0
        self._load_states(g["in"], states)
        g["graph"].replay()
        mk = self._persistent(B, 1)
        if mk is not None:
            mk.check_deferred(torch.cuda.current_stream(self.device))
        new = [(s.clone(), t.clone(), c.clone()) for s, t, c in g["out"]]
        return g["logits"].clone().reshape(B, 1, -1), new

    def _capture(self, B):
        """Two graphs of one decode step over static buffers: graph 0 reads
        state set 0 and writes set 1, graph 1 the reverse, so a replayed
        token stream carries its state without copies."""
        dev = self.device
        idx = torch.zeros(B, 1, dtype=torch.int64, device=dev)
        sets = [self._new_states(B), self._new_states(B)]
        for st in sets:
            for s in st:
                for t in s:
                    t.zero_()
        wk = self._work_for(B)
        logits = torch.empty(B, self.vocab_size, device=dev)

        def run(src, dst):
            self._body(idx, src, wk, dst)
            _apply(self.head, wk.xo, logits, _lib.EPI_STORE)

        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            run(sets[0], sets[1])           # warm-up outside the graph
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        mk = self._persistent(B, 1)
        if mk is not None:               # descriptor tables, both directions
            mk.prepare(sets[0], sets[1], wk)
            mk.prepare(sets[1], sets[0], wk)
        graphs = []
        for k in range(2):
            gph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gph):
                run(sets[k], sets[1 - k])
            graphs.append(gph)
        torch.cuda.synchronize(dev)
        for st in sets:
            for s in st:
                for t in s:
                    t.zero_()
        return {"graphs": graphs, "idx": idx, "sets": sets, "logits": logits,
                "next": 0, "in": sets[0], "out": sets[1],
                "graph": graphs[0]}

    def decode_replay(self, B, ids=None):
        """Benchmark/serving hook: one decode step of batch B on the
        captured graphs, carrying the state in the static buffers
        (ping-pong).  `ids` (device int64 [B]) is copied into the input
        slot first.  Returns the static logits buffer [B, V]."""
        g = self._graphs.get(B)
        if g is None:
            g = self._capture(B)
            self._graphs[B] = g
        if ids is not None:
            g["idx"].copy_(ids.reshape(B, 1))
        g["graphs"][g["next"]].replay()
        g["next"] ^= 1
        return g["logits"]

    def reset_replay_state(self, B):
        g = self._graphs.get(B)
        if g is None:
            return
        for st in g["sets"]:
            for s in st:
                for t in s:
                    t.zero_()
        g["next"] = 0
