"""Block (group-wise) quantizers that produce the codes stored in `.rwkvq`.

These decide which integers land in the file; the HIP kernels only read
them.  The arithmetic must match the reference quantizer step for step,
because the reference freezes SHA-256 digests of the outputs
(reference: tests/make_gw_golden.py:62-118, tests/fixtures/gw_golden.json)
and the packers build the on-disk fields straight from these parts.

Public names and signatures mirror the reference module
(reference: rwkv_quant/calibration/groupwise.py:153-176, 308-355) so that
writer code and tests can call them the same way:

    groupwise_fake_dequant(w, bits, gs, sb=0, sb_bits=6, ex2=None,
                           return_parts=False)
    groupwise_sym_fake_dequant(w, bits, gs=16, sb=16, ex2=None,
                               search=True, outlier_frac=0.0,
                               return_parts=False)

Both work on row bands: every quantity is computed inside one row, so the
band split changes no bit (reference: groupwise.py:163-170).
"""
import os

import torch
import torch.nn.functional as F

__all__ = ["groupwise_fake_dequant", "groupwise_sym_fake_dequant",
           "GW_MODES", "mode_needs_act_stats", "get_ex2"]

# mode name -> (needs activation statistics, description)
# (reference: groupwise.py:40-49)
GW_MODES = {
    "asym": (False, "asymmetric RTN per block, no superblock"),
    "asym_sb6": (False, "sb6 superblock, no scale search"),
    "asym_sb6_search": (False, "sb6 + grid/LS search of scale/min"),
    "asym_sb6_aw": (True, "sb6 + search weighted by E[x^2]"),
    "sym": (False, "Q6_K-style symmetric layout + scale search"),
    "sym_plain": (False, "Q6_K-style symmetric layout, no search"),
    "sym_aw": (True, "symmetric, search weighted by E[x^2]"),
}

# grid factors of the asymmetric search (reference: groupwise.py:237)
_ASYM_FACTORS = (0.7, 0.75, 0.8, 0.85, 0.9, 0.95, 1.0, 1.05)
# 19 float32 nodes of linspace(0.7, 1.15), materialised as Python floats
# (reference: groupwise.py:305)
_SYM_FACTORS = tuple(torch.linspace(0.7, 1.15, 19).tolist())

# row-band budget in bytes of fp32 input (reference: groupwise.py:150)
_BAND_BYTES = int(os.environ.get("RWKVQ_GW_CHUNK_MB", "128")) << 20


def mode_needs_act_stats(mode: str) -> bool:
    return GW_MODES.get(mode, (False, ""))[0]


def get_ex2(path, key, w):
    """Activation statistics are an offline calibration artefact; without a
    stats file every AW mode degrades to its unweighted search, exactly as
    the reference does when the file is absent
    (reference: groupwise.py:63-129)."""
    if not path or key is None or not os.path.exists(path):
        return None
    stats = torch.load(path, weights_only=True)
    ex2 = stats.get(key)
    if ex2 is None or ex2.numel() != w.shape[-1]:
        return None
    return ex2


def _bands(n_rows, n_cols):
    per = max(1, _BAND_BYTES // max(1, n_cols * 4))
    return [(r, min(n_rows, r + per)) for r in range(0, n_rows, per)]


def _run_banded(fn, w, ex2, return_parts, *args):
    if w.dim() != 2 or (ex2 is not None and ex2.dim() > 1):
        return fn(w, *args)
    bands = _bands(w.shape[0], w.shape[1])
    if len(bands) == 1:
        return fn(w, *args)
    outs = [fn(w[a:b], *args) for a, b in bands]
    if return_parts:
        return {k: torch.cat([o[k] for o in outs], dim=0) for k in outs[0]}
    return torch.cat(outs, dim=0)


# ---------------------------------------------------------------- asymmetric

def groupwise_fake_dequant(w, bits, gs, sb=0, sb_bits=6, ex2=None,
                           return_parts=False):
    """Asymmetric block RTN (scale + min per block of `gs` columns); with
    `sb` the block scales/mins are themselves quantized in `|sb_bits|` bits
    against one fp16 pair (d, dm) per superblock of `sb` blocks; a negative
    `sb_bits` first runs the grid + least-squares search of (scale, min).
    Returns the dequantized weight, or its parts for the packer.
    (reference: groupwise.py:153-300)"""
    return _run_banded(_asym_band, w, ex2, return_parts,
                       bits, gs, sb, sb_bits, ex2, return_parts)


def _ls_fit(wg, qq, evg):
    """Closed-form least squares of w ~ q*s + m on each block, optionally
    weighted by evg (reference: groupwise.py:240-251)."""
    if evg is None:
        q_mean = qq.mean(dim=2, keepdim=True)
        w_mean = wg.mean(dim=2, keepdim=True)
        cov = ((qq - q_mean) * (wg - w_mean)).sum(dim=2, keepdim=True)
        var = ((qq - q_mean) ** 2).sum(dim=2, keepdim=True).clamp_min(1e-12)
    else:
        wsum = evg.sum(dim=2, keepdim=True)
        q_mean = (evg * qq).sum(dim=2, keepdim=True) / wsum
        w_mean = (evg * wg).sum(dim=2, keepdim=True) / wsum
        cov = (evg * (qq - q_mean) * (wg - w_mean)).sum(dim=2, keepdim=True)
        var = (evg * (qq - q_mean) ** 2).sum(dim=2,
                                              keepdim=True).clamp_min(1e-12)
    s = cov / var
    return s, w_mean - s * q_mean


def _asym_band(w, bits, gs, sb, sb_bits, ex2, return_parts):
    w32 = w.float()
    n_out, n_in = w32.shape
    pad = (-n_in) % gs
    wp = F.pad(w32, (0, pad)) if pad else w32
    nb = wp.shape[1] // gs
    wg = wp.view(n_out, nb, gs)
    lo = wg.amin(dim=2, keepdim=True)
    hi = wg.amax(dim=2, keepdim=True)
    qmax = 2 ** bits - 1
    scale = ((hi - lo) / qmax).clamp_min(1e-8)
    mn = lo
    evg = None
    if ex2 is not None:
        ev = ex2.to(w32.device).float().clamp_min(1e-12)
        evg = (F.pad(ev, (0, pad)) if pad else ev).view(1, nb, gs)

    if sb and sb_bits < 0:
        best_s = best_m = best_e = None
        for f in _ASYM_FACTORS:
            trial = scale * f
            qq = torch.clamp(torch.round((wg - lo) / trial), 0, qmax)
            s_ls, m_ls = _ls_fit(wg, qq, evg)
            s_ls = torch.where(s_ls > 1e-8, s_ls, trial)
            q2 = torch.clamp(torch.round((wg - m_ls) / s_ls), 0, qmax)
            e2 = (q2 * s_ls + m_ls - wg) ** 2
            err = (e2 if evg is None else evg * e2).sum(dim=2, keepdim=True)
            if best_e is None:
                best_s, best_m, best_e = s_ls, m_ls, err
            else:
                better = err < best_e
                best_s = torch.where(better, s_ls, best_s)
                best_m = torch.where(better, m_ls, best_m)
                best_e = torch.minimum(best_e, err)
        scale, mn = best_s.clamp_min(1e-8), best_m
        sb_bits = -sb_bits

    parts_sb = None
    if sb:
        # superblock quantization of the block scales / mins; d and dm pass
        # the fp16 round trip BEFORE qs/qm are chosen, so the kernel rebuilds
        # s = half(qs * d) bit for bit (reference: groupwise.py:265-289)
        pad_b = (-nb) % sb
        s_pad = F.pad(scale, (0, 0, 0, pad_b)) if pad_b else scale
        m_pad = F.pad(mn, (0, 0, 0, pad_b)) if pad_b else mn
        ssb = s_pad.view(n_out, -1, sb, 1)
        msb = m_pad.view(n_out, -1, sb, 1)
        smax = 2 ** sb_bits - 1
        d = (ssb.amax(dim=2, keepdim=True) / smax).clamp_min(1e-12) \
            .half().float()
        qs = torch.clamp(torch.round(ssb / d), 1, smax)
        mmax = 2 ** (sb_bits - 1) - 1
        dm = (msb.abs().amax(dim=2, keepdim=True) / mmax).clamp_min(1e-12) \
            .half().float()
        qm = torch.clamp(torch.round(msb / dm), -mmax, mmax)
        s_q = (qs * d).view(n_out, -1, 1)[:, :nb]
        m_q = (qm * dm).view(n_out, -1, 1)[:, :nb]
        # fp16 underflow of near-constant blocks would make 0/0 codes
        scale = s_q.half().float().clamp_min(1e-8)
        mn = m_q.half().float()
        parts_sb = (qs, qm, d, dm)

    qv = torch.clamp(torch.round((wg - mn) / scale), 0, qmax)
    deq = (qv * scale + mn).view(n_out, -1)[:, :n_in]
    if not return_parts:
        return deq
    parts = {"q": qv.view(n_out, -1)[:, :n_in].to(torch.uint8), "deq": deq,
             "scale": scale, "mn": mn}
    if parts_sb is not None:
        qs, qm, d, dm = parts_sb
        parts["qs"] = qs.view(n_out, -1)[:, :nb].to(torch.uint8)
        parts["qm"] = qm.view(n_out, -1)[:, :nb].to(torch.int8)
        parts["d"] = d.view(n_out, -1).half()
        parts["dm"] = dm.view(n_out, -1).half()
    return parts


# ----------------------------------------------------------------- symmetric

def groupwise_sym_fake_dequant(w, bits, gs=16, sb=16, ex2=None, search=True,
                               outlier_frac=0.0, return_parts=False):
    """Q6_K-style symmetric blocks: one scale per `gs` weights, no min; the
    block scales are int8 codes against one fp16 `d` per superblock of `sb`
    blocks.  `search` scans 19 scale factors; `outlier_frac` keeps the top
    |w| of each row exact (fake path only).
    (reference: groupwise.py:308-473)"""
    return _run_banded(_sym_band, w, ex2, return_parts,
                       bits, gs, sb, ex2, search, outlier_frac, return_parts)


def _sym_band(w, bits, gs, sb, ex2, search, outlier_frac, return_parts):
    w32 = w.float()
    n_out, n_in = w32.shape
    omask = None
    body = w32
    if outlier_frac > 0.0:
        k = max(1, int(round(n_in * outlier_frac)))
        kth = torch.topk(w32.abs(), k, dim=1).values[:, -1:].clamp_min(1e-20)
        omask = w32.abs() >= kth
        body = torch.where(omask, torch.zeros_like(w32), w32)
    pad = (-n_in) % (gs * sb)
    wp = F.pad(body, (0, pad)) if pad else body
    nb = wp.shape[1] // gs
    wg = wp.view(n_out, nb, gs)
    evg = None
    if ex2 is not None:
        ev = ex2.to(w32.device).float().clamp_min(1e-12).view(1, -1)
        evg = (F.pad(ev, (0, pad)) if pad else ev).view(1, nb, gs)

    qmax = 2 ** (bits - 1) - 1
    qmin = -qmax - 1
    base = wg.abs().amax(dim=2, keepdim=True).clamp_min(1e-12) / qmax
    best_s = best_e = None
    for f in (_SYM_FACTORS if search else (1.0,)):
        s = base * f
        qv = torch.clamp(torch.round(wg / s), qmin, qmax)
        e = (wg - qv * s) ** 2
        err = (e if evg is None else evg * e).sum(dim=2, keepdim=True)
        if best_e is None:
            best_s, best_e = s, err
        else:
            better = err < best_e
            best_s = torch.where(better, s, best_s)
            best_e = torch.minimum(best_e, err)

    ssb = best_s.view(n_out, -1, sb, 1)
    d = (ssb.amax(dim=2, keepdim=True) / 127.0).clamp_min(1e-12).half() \
        .float()
    qs = torch.clamp(torch.round(ssb / d), -128, 127)
    scale_q = (qs * d).view(n_out, nb, 1).half().float()
    nz = scale_q.abs() > 0
    qv = torch.clamp(torch.round(wg / torch.where(nz, scale_q,
                                                  torch.ones_like(scale_q))),
                     qmin, qmax)
    qv = torch.where(nz, qv, torch.zeros_like(qv))
    deq = (qv * scale_q).view(n_out, -1)[:, :n_in]
    if omask is not None:
        deq = torch.where(omask, w32, deq)
    if not return_parts:
        return deq
    # a degenerate superblock (all zero) makes qs = 0/0; the file stores 0
    # there, which dequantizes to exactly the zeros of `deq`
    # (reference: groupwise.py:462-473)
    return {"deq": deq,
            "q": qv.view(n_out, -1).to(torch.int8),
            "qs": torch.nan_to_num(qs, 0.0).view(n_out, nb).to(torch.int8),
            "d": d.view(n_out, -1).half()}
