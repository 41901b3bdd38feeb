"""Perplexity harness on the GPU (reference: rwkv_quant/calibration/
ablation.py:21-69).

`perplexity(model, data, cfg=None, batch_size=2)` has the reference's
semantics: rows of `data` [n_chunks, chunk_len] are independent sequences,
batch_size rows at a time run through the model from a zero state, the
logits of data[:, :-1] are scored against data[:, 1:] with
NLL = logsumexp(logits) - logit[target], and the result is
exp(mean NLL over every scored token).  A degenerate mean (not finite or
<= 1e-6) raises instead of returning a number that looks like a result.

The model is the HIP backend's QuantRWKV7: its weights are the file's real
quantized codes, so there is nothing left for a fake-quant `cfg` to do
(the reference's cfg drives RWKV7Ref's fake quantization); a cfg that asks
for quantization raises.  The per-row NLL is a librwkvq_hip kernel
(rwkvq_nll_rows); only the per-batch sum of the NLL rows is added up on the
host, in float64.
"""
import math

import torch

from ..backends.hip import _lib


def nll_rows(logits, targets):
    """logits [..., V] fp32 on the GPU, targets [...] int -> nll [...]
    (rwkvq_nll_rows)."""
    V = logits.shape[-1]
    lg = logits.reshape(-1, V)
    if lg.stride(-1) != 1 or lg.dtype != torch.float32:
        lg = lg.float().contiguous()
    tg = targets.reshape(-1).to(device=lg.device, dtype=torch.int64) \
        .contiguous()
    if tg.numel() != lg.shape[0]:
        raise ValueError(f"{tg.numel()} targets for {lg.shape[0]} rows")
    out = torch.empty(lg.shape[0], dtype=torch.float32, device=lg.device)
    _lib.call("rwkvq_nll_rows", _lib.ptr(lg), lg.stride(0), _lib.ptr(tg),
              lg.shape[0], V, _lib.ptr(out), _lib.stream_handle())
    return out.reshape(targets.shape)


def _check_cfg(cfg):
    if cfg is None:
        return
    bits = getattr(cfg, "bits", {})
    if any(b < 16 for b in bits.values()):
        raise ValueError("perplexity on a HIP QuantRWKV7: the model already "
                         "holds quantized weights; pass cfg=None")


def finish(total_nll, total_tok):
    """exp(mean NLL), refusing a degenerate mean (reference:
    ablation.py:51-69)."""
    mean_nll = total_nll / max(total_tok, 1)
    if not math.isfinite(mean_nll) or mean_nll <= 1e-6:
        raise RuntimeError(
            f"degenerate perplexity (mean NLL = {mean_nll!r}): the logits "
            f"were not computed; check the device logs and the batch size")
    return math.exp(mean_nll)


@torch.no_grad()
def perplexity(model, data, cfg=None, batch_size=2):
    """exp(mean next-token NLL) of `model` over the rows of `data`."""
    _check_cfg(cfg)
    data = torch.as_tensor(data)
    if data.dim() != 2 or data.shape[1] < 2:
        raise ValueError("data must be [n_chunks, chunk_len >= 2]")
    total_nll, total_tok = 0.0, 0
    for i in range(0, data.shape[0], batch_size):
        batch = data[i:i + batch_size]
        logits, _ = model.forward_stateful(batch[:, :-1],
                                           model.init_state(batch.shape[0]))
        nll = nll_rows(logits, batch[:, 1:])
        total_nll += float(nll.cpu().double().sum())
        total_tok += nll.numel()
        del logits, nll
    return finish(total_nll, total_tok)
