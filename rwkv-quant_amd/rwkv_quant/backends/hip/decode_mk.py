"""Host side of the persistent decode kernel (rwkvq_decode_mk): the layer
descriptor table of a QuantRWKV7 and the launch.

One batch-1 decode step runs as: embedding gather + ln0, ONE launch for
every layer (five phases per layer separated by grid barriers inside the
kernel), ln_out, head.  The per-layer math is the decode body of the
reference (reference: rwkv_quant/backends/metal/quant_model.py:638-728,
803-809), the same as the per-kernel path of QuantRWKV7._body.

The descriptor mirrors `struct MkLayer` of csrc/decode_mk.hip field for
field; its size is checked against rwkvq_decode_mk_info.  A table holds the
state pointers of one (input states, output states) pair, so the two
ping-pong directions of a captured decode graph have one table each; tables
are built outside stream capture (an H2D copy) and cached.
"""
import ctypes
from collections import OrderedDict

import torch

from . import _lib
from .quant_linear import (GwQuantLinear, GwQuantLinearFused, SymQuantLinear,
                           SymQuantLinearFused)

_P = ctypes.c_void_p
_I = ctypes.c_int

F_SB6_4, F_SB6_5, F_SYM6, F_SYM8 = 0, 1, 3, 4
FORMAT_PAIRS = ((F_SB6_5, F_SB6_4), (F_SYM8, F_SYM6))
DOWN_ROWS_PER_WG = 8            # LoRA down rows per workgroup (2 per wave)
DOWN_WGS = 64                   # workgroups left for them beside r/k/v
MAX_TABLES = 4
MAX_RANK = 256                  # one rank position per thread of a workgroup


class MkMat(ctypes.Structure):
    _fields_ = [("q", _P), ("hb", _P), ("rec", _P), ("qs", _P), ("d", _P),
                ("rows", _I), ("in_", _I)]


class MkDown(ctypes.Structure):
    _fields_ = [("q", _P), ("s", _P), ("m", _P), ("sc", _P), ("y", _P),
                ("rows", _I), ("slot", _I), ("epi", _I), ("wg0", _I)]


class MkUp(ctypes.Structure):
    _fields_ = [("h", _P * 4), ("q", _P * 4), ("s", _P * 4), ("m", _P * 4),
                ("sc", _P * 4), ("r", _I * 4)]


class MkLayer(ctypes.Structure):
    _fields_ = [("rkv", MkMat), ("o", MkMat), ("key", MkMat), ("val", MkMat),
                ("ln1_w", _P), ("ln1_b", _P), ("coef", _P),
                ("tshift_in", _P), ("tshift_out", _P),
                ("ln2_w", _P), ("ln2_b", _P), ("xk", _P),
                ("cshift_in", _P), ("cshift_out", _P),
                ("down", MkDown * 4), ("up", MkUp),
                ("w0", _P), ("a0", _P), ("v0", _P), ("k_k", _P), ("k_a", _P),
                ("r_k", _P), ("lnx_w", _P), ("lnx_b", _P),
                ("state_in", _P), ("state_out", _P),
                ("n_down", _I), ("layer0", _I), ("lora_wgs", _I),
                ("pad", _I)]


def _p(t):
    return None if t is None else t.data_ptr()


def _fmt(lin):
    """Kernel format id of a GEMV operand (None if not supported here)."""
    if isinstance(lin, (GwQuantLinear, GwQuantLinearFused)):
        b = lin.bits
        return {4: F_SB6_4, 5: F_SB6_5}.get(b)
    if isinstance(lin, (SymQuantLinear, SymQuantLinearFused)):
        return {6: F_SYM6, 8: F_SYM8}.get(lin.bits)
    return None


def _mat(lin):
    c = getattr(lin, "_cat", lin)
    m = MkMat()
    if isinstance(c, GwQuantLinear):
        m.q, m.hb, m.rec = _p(c.nib), _p(c.hb), _p(c.rec)
    else:
        m.q, m.hb, m.qs, m.d = _p(c.codes), _p(c.hb), _p(c.qs), _p(c.d)
    m.rows, m.in_ = c.out_features, c.in_features
    return m


class PersistentDecode:
    """rwkvq_decode_mk for one model; `ok` is False when the model's shape,
    formats or LoRA layout are outside what the kernel covers."""

    def __init__(self, model):
        self.model = model
        self.ok = False
        self.why = ""
        lb, bw, wgs, max_cat = (ctypes.c_int(), ctypes.c_int(),
                                ctypes.c_int(), ctypes.c_int())
        _lib.call("rwkvq_decode_mk_info", ctypes.byref(lb), ctypes.byref(bw),
                  ctypes.byref(wgs), ctypes.byref(max_cat))
        if lb.value != ctypes.sizeof(MkLayer):
            raise _lib.HipKernelError(
                f"MkLayer is {ctypes.sizeof(MkLayer)} bytes here, "
                f"{lb.value} in the library")
        self.bar_words, self.max_cat = bw.value, max_cat.value
        self.why = self._check()
        if self.why:
            return
        dev = model.device
        self.bar = torch.zeros(self.bar_words, dtype=torch.int32, device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        # activation arena: one region per (layer, phase output), written
        # once per launch (the kernel reads them through the L2), and the
        # LoRA down outputs, one 128-byte aligned region per layer
        D, F, L = model.n_embd, model.ffn, model.n_layer
        self.act_stride = 6 * D + F
        self.act = torch.zeros(L * self.act_stride, dtype=torch.float32,
                               device=dev)
        self.h_off, off = [], 0
        for blk in model.blocks:
            offs = {}
            for b in blk.tmix.lora_q:
                offs[b] = off
                off += -(-blk.tmix.lora_q[b][0] // 32) * 32
            self.h_off.append(offs)
        self.hbuf = torch.zeros(max(off, 32), dtype=torch.float32, device=dev)
        self.fmts = (_fmt(model.blocks[0].tmix.rkv_fused),
                     _fmt(model.blocks[0].cmix.key))
        self._tables = OrderedDict()
        self.ok = True

    def _check(self):
        m = self.model
        if m.n_embd != 2048 or m.ffn != 4 * m.n_embd or m.head_size != 64:
            return "shape (D 2048, F 4 D, head 64 only)"
        pair = None
        for blk in m.blocks:
            tm, cm = blk.tmix, blk.cmix
            if tm.rkv_fused is None or tm.lora_q is None:
                return "r/k/v not fused or LoRA not read from codes"
            f = (_fmt(tm.rkv_fused), _fmt(cm.key))
            if f not in FORMAT_PAIRS or _fmt(tm.o_proj) != f[0] or \
                    _fmt(cm.value) != f[1]:
                return f"formats {f}"
            if pair not in (None, f):
                return "formats differ between layers"
            pair = f
            ranks = [tm.lora_q[b][0] for b in tm.lora_q]
            # the WKV phase stages one rank position per thread (256)
            if any(r % 16 or r > MAX_RANK for r in ranks) or \
                    sum(ranks) > self.max_cat:
                return "LoRA ranks"
            if sum(-(-r // DOWN_ROWS_PER_WG) for r in ranks) > DOWN_WGS:
                return "LoRA down rows"
        return ""

    def _table(self, states, out_states, wk):
        """Device descriptor table for this (states, out_states) pair."""
        key = tuple(_p(t) or 0 for s in list(states) + list(out_states)
                    for t in s) + (wk.x.data_ptr(),)
        t = self._tables.get(key)
        if t is not None:
            self._tables.move_to_end(key)
            return t
        if torch.cuda.is_current_stream_capturing():
            raise _lib.HipKernelError(
                "persistent decode: descriptor table built during capture")
        m = self.model
        arr = (MkLayer * m.n_layer)()
        for li, (blk, st, so) in enumerate(zip(m.blocks, states, out_states)):
            tm, cm = blk.tmix, blk.cmix
            L = arr[li]
            L.rkv, L.o = _mat(tm.rkv_fused), _mat(tm.o_proj)
            L.key, L.val = _mat(cm.key), _mat(cm.value)
            L.ln1_w, L.ln1_b = _p(blk.ln1_w), _p(blk.ln1_b)
            L.coef = _p(tm.coef)
            L.tshift_in, L.tshift_out = _p(st[1]), _p(so[1])
            L.ln2_w, L.ln2_b = _p(blk.ln2_w), _p(blk.ln2_b)
            L.xk = _p(cm.x_k)
            L.cshift_in, L.cshift_out = _p(st[2]), _p(so[2])
            wg0 = 0
            for j, b in enumerate(tm.lora_q):
                rank, dn, _ = tm.lora_q[b]
                d = L.down[j]
                d.q, d.s, d.m, d.sc = (_p(dn["q"]), _p(dn["s"]), _p(dn["m"]),
                                       _p(dn["sc"]))
                d.y = self.hbuf.data_ptr() + 4 * self.h_off[li][b]
                d.rows, d.slot, d.epi, d.wg0 = (rank, tm.SLOT[b],
                                                tm.EPI_DOWN[b], wg0)
                wg0 += -(-rank // DOWN_ROWS_PER_WG)
            L.n_down, L.lora_wgs = len(tm.lora_q), wg0
            for k, b in enumerate(("w", "a", "v", "g")):
                if b not in tm.lora_q:
                    continue
                rank, _, up = tm.lora_q[b]
                L.up.h[k] = self.hbuf.data_ptr() + 4 * self.h_off[li][b]
                L.up.q[k], L.up.s[k] = _p(up["q"]), _p(up["s"])
                L.up.m[k], L.up.sc[k] = _p(up["m"]), _p(up["sc"])
                L.up.r[k] = rank
            L.w0, L.a0, L.v0 = _p(tm.w0), _p(tm.a0), _p(tm.v0)
            L.k_k, L.k_a, L.r_k = _p(tm.k_k), _p(tm.k_a), _p(tm.r_k)
            L.lnx_w, L.lnx_b = _p(tm.ln_x_w), _p(tm.ln_x_b)
            L.state_in, L.state_out = _p(st[0]), _p(so[0])
            L.layer0 = 1 if li == 0 else 0
        raw = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
        t = raw.to(m.device)
        torch.cuda.synchronize(m.device)
        self._tables[key] = t
        while len(self._tables) > MAX_TABLES:
            self._tables.popitem(last=False)
        return t

    def prepare(self, states, out_states, wk):
        """Build (outside capture) the table a later captured step uses."""
        self._table(states, out_states, wk)

    def run(self, states, out_states, wk, stream):
        """The layers of one batch-1 decode step: wk.x (after ln0) in,
        wk.x (before ln_out) out; new states written to out_states."""
        m = self.model
        t = self._table(states, out_states, wk)
        _lib.call("rwkvq_decode_mk", _lib.ptr(t), m.n_layer, self.fmts[0],
                  self.fmts[1], m.n_embd, m.ffn, m.n_head, _lib.ptr(wk.x),
                  _lib.ptr(self.act), self.act.numel(), _lib.ptr(wk.v_first),
                  _lib.ptr(self.bar), _lib.ptr(self.err), stream)

    def error_flag(self):
        """True when some launch's barrier wait ran past its limit (a
        synchronizing read)."""
        return bool(self.err.item())

    def check_deferred(self, stream):
        """Raise if a launch checked by an earlier call set the error flag;
        then queue an asynchronous copy of the flag for the next call.  No
        synchronization: a launch is seen by the call after the copy has
        landed (the flag is sticky, so a violation is never missed for
        long).  A set flag means that not every workgroup was resident at
        once -- the kernel must not share the device with concurrent work --
        and that launch's results are invalid."""
        if getattr(self, "_err_host", None) is None:
            self._err_host = torch.zeros(1, dtype=torch.int32,
                                         pin_memory=True)
        elif int(self._err_host[0]):
            raise _lib.HipKernelError(
                "persistent decode: a grid-barrier wait ran past its limit "
                "(not every workgroup was resident; concurrent kernels on "
                "the device?) -- decode results are invalid")
        with torch.cuda.stream(stream):
            self._err_host.copy_(self.err, non_blocking=True)
