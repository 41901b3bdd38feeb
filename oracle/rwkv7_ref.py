"""TEST INFRASTRUCTURE ONLY -- CPU oracle of the RWKV-7 forward.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s cpu_baseline may
import this; the product never does.

A float64 numpy restatement of the reference forward
(reference: rwkv_quant/models/rwkv7_ref.py:184-290) with the stateful
streaming semantics of the inference model (reference:
rwkv_quant/backends/metal/quant_model.py:292-301, 827-836, 902-990):
per-layer state (wkv [B, H, N, N], time-mix shift, channel-mix shift),
shift = 0 on the first call.  Weights are the oracle's exact dequant of the
checkpoint (codec_ref.dequant_qt), world LoRA transposed after dequant
(reference: rwkv_quant/formats/codec.py:514-535).

Pinned (tests/test_reference_fixtures.py) against the reference's own
RWKV7Ref forward (fp32, CPU) on a seeded 3-layer model: logits and the
residual stream after every block within 1e-5 relative, and its
`perplexity` (calibration/ablation.py:21-69); each of a wrong group-norm
eps, a bonus without r_k, the output gate's sigmoid after the up product
and a missing v-residual, planted in a subclass, fails that check.  Also
pinned by properties (tests/test_oracle_forward.py): token-by-token ==
whole-sequence, the w = 1, a = b = 0 case equals the closed-form
linear-attention sum, the decay identity exp(-exp(-softplus(-z) - 0.5)) ==
exp(-0.606531 sigmoid(z)), and a brute-force per-element recurrence on a
tiny head.
"""
import numpy as np

from . import codec_ref

_LORA = ("w1", "w2", "a1", "a2", "v1", "v2", "g1", "g2")


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _softplus(x):
    return np.logaddexp(0.0, x)


def layer_norm(x, w, b, eps=1e-5):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * w + b


def group_norm(x, H, w, b, eps=64e-5):
    sh = x.shape
    xg = x.reshape(sh[:-1] + (H, -1))
    m = xg.mean(-1, keepdims=True)
    v = ((xg - m) ** 2).mean(-1, keepdims=True)
    return ((xg - m) / np.sqrt(v + eps)).reshape(sh) * w + b


def wkv7(r, w, k, v, a, b, state):
    """Recurrence per (batch, head), as rwkv7_ref._wkv7 but from a given
    state: S = S diag(w) + (S a) b^T + v k^T; y = S r.  Inputs [B, T, H, N]
    (w is the decay itself); state [B, H, N, N]; returns (y, new state)."""
    B, T, H, N = r.shape
    S = state.astype(np.float64).copy()
    y = np.zeros((B, T, H, N))
    for t in range(T):
        sa = np.einsum("bhij,bhj->bhi", S, a[:, t])
        S = S * w[:, t, :, None, :] + sa[..., None] * b[:, t, :, None, :] \
            + v[:, t, :, :, None] * k[:, t, :, None, :]
        y[:, t] = np.einsum("bhij,bhj->bhi", S, r[:, t])
    return y, S


class RWKV7Oracle:
    def __init__(self, ckpt):
        self.naming = ckpt.naming
        self.n_layer, self.C = ckpt.n_layer, ckpt.n_embd
        self.N = ckpt.head_size
        self.H = self.C // self.N
        world = ckpt.naming == "world"
        self.p = {}
        for key, qt in ckpt.tensors.items():
            a = codec_ref.dequant_qt(qt).astype(np.float64)
            if world and key.split(".")[-1] in _LORA:
                a = a.T.copy()        # stored [in, out]: dequant, then .T
            self.p[key] = a

    def init_state(self, B):
        return [(np.zeros((B, self.H, self.N, self.N)), None, None)
                for _ in range(self.n_layer)]

    def _g(self, name):
        return self.p[name]

    @staticmethod
    def _shift(x, prev):
        B, T, C = x.shape
        first = np.zeros((B, 1, C)) if prev is None else prev.reshape(B, 1, C)
        return np.concatenate([first, x[:, :-1]], axis=1), x[:, -1].copy()

    # The time mix is split into the steps below so that a test can plant
    # a mistake in one of them (a subclass overriding it) and show that
    # the reference fixture catches it.
    def _v_residual(self, i, v, v_first, xv):
        """v + (v_first - v) sigmoid(xv A_v^T B_v^T + v0), layers > 0
        (reference: rwkv7_ref.py:203-208)."""
        g = lambda s: self._g(f"blocks.{i}.att.{s}")
        gate = _sigmoid(xv @ g("v1").T @ g("v2").T + g("v0").reshape(-1))
        return v + (v_first - v) * gate

    def _gate(self, i, xg):
        """sigmoid(xg A_g^T) B_g^T (reference: rwkv7_ref.py:212)."""
        g = lambda s: self._g(f"blocks.{i}.att.{s}")
        return _sigmoid(xg @ g("g1").T) @ g("g2").T

    def _bonus(self, i, r, k, v):
        """(sum_n r k r_k) v per head, inputs [B, T, H, N]
        (reference: rwkv7_ref.py:226-228)."""
        r_k = self._g(f"blocks.{i}.att.r_k").reshape(self.H, self.N)
        return (r * k * r_k).sum(-1, keepdims=True) * v

    def _norm_out(self, i, y):
        """Per-head group norm, eps 64e-5 (reference: rwkv7_ref.py:223-224)."""
        g = lambda s: self._g(f"blocks.{i}.att.{s}")
        return group_norm(y, self.H, g("ln_x.weight"), g("ln_x.bias"))

    def _tmix(self, i, x, v_first, state):
        g = lambda s: self._g(f"blocks.{i}.att.{s}")
        B, T, C = x.shape
        H, N = self.H, self.N
        wkv_state, prev = state
        sx, new_prev = self._shift(x, prev)
        xx = sx - x
        lerp = lambda s: x + xx * g(s).reshape(C)
        xr, xw, xk, xv, xa, xg = (lerp(s) for s in
                                  ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"))
        r = xr @ g("receptance.weight").T
        k = xk @ g("key.weight").T
        v = xv @ g("value.weight").T
        # A matrices are [r, C] (w1.T), B matrices [C, r] (w2.T)
        w_ = -_softplus(-(np.tanh(xw @ g("w1").T) @ g("w2").T
                          + g("w0").reshape(C))) - 0.5
        if i == 0:
            v_first = v
        else:
            v = self._v_residual(i, v, v_first, xv)
        a = _sigmoid(xa @ g("a1").T @ g("a2").T + g("a0").reshape(C))
        gg = self._gate(i, xg)
        kk = (k * g("k_k").reshape(C)).reshape(B, T, H, N)
        kk = kk / np.maximum(np.linalg.norm(kk, axis=-1, keepdims=True),
                             1e-12)
        kk = kk.reshape(B, T, C)
        k = k * (1 + (a - 1) * g("k_a").reshape(C))
        w = np.exp(-np.exp(w_))
        sh = (B, T, H, N)
        y, new_state = wkv7(r.reshape(sh), w.reshape(sh), k.reshape(sh),
                            v.reshape(sh), (-kk).reshape(sh),
                            (kk * a).reshape(sh), wkv_state)
        out = self._norm_out(i, y.reshape(B, T, C))
        bonus = self._bonus(i, r.reshape(sh), k.reshape(sh),
                            v.reshape(sh)).reshape(B, T, C)
        out = (out + bonus) * gg
        return out @ g("output.weight").T, v_first, (new_state, new_prev)

    def _cmix(self, i, x, prev):
        g = lambda s: self._g(f"blocks.{i}.ffn.{s}")
        sx, new_prev = self._shift(x, prev)
        xk = x + (sx - x) * g("x_k").reshape(-1)
        h = np.maximum(xk @ g("key.weight").T, 0.0) ** 2
        return h @ g("value.weight").T, new_prev

    def forward_stateful(self, idx, states, hidden_only=False, trace=None):
        """trace: a list that receives the residual stream after every
        block, as the reference's `trace` argument (rwkv7_ref.py:261-283)."""
        idx = np.asarray(idx)
        x = self._g("emb.weight")[idx]
        x = layer_norm(x, self._g("blocks.0.ln0.weight"),
                       self._g("blocks.0.ln0.bias"))
        v_first = None
        new_states = []
        for i, (wkv_s, tshift, cshift) in enumerate(states):
            p = f"blocks.{i}."
            xn = layer_norm(x, self._g(p + "ln1.weight"),
                            self._g(p + "ln1.bias"))
            att, v_first, (ns, nt) = self._tmix(i, xn, v_first,
                                                (wkv_s, tshift))
            x = x + att
            xn2 = layer_norm(x, self._g(p + "ln2.weight"),
                             self._g(p + "ln2.bias"))
            ff, nc = self._cmix(i, xn2, cshift)
            x = x + ff
            new_states.append((ns, nt, nc))
            if trace is not None:
                trace.append(x.copy())
        x = layer_norm(x, self._g("ln_out.weight"), self._g("ln_out.bias"))
        if hidden_only:
            return x, new_states
        return x @ self._g("head.weight").T, new_states


def perplexity(orc, data, batch_size=2):
    """exp(mean NLL) of next-token prediction over rows of `data` [n, L],
    each row a fresh sequence (reference: calibration/ablation.py:21-69:
    logits of data[:, :-1], NLL = logsumexp - logit[target])."""
    data = np.asarray(data)
    tot, cnt = 0.0, 0
    for i in range(0, data.shape[0], batch_size):
        batch = data[i:i + batch_size]
        lg, _ = orc.forward_stateful(batch[:, :-1],
                                     orc.init_state(batch.shape[0]))
        m = lg.max(-1, keepdims=True)
        lse = (m + np.log(np.exp(lg - m).sum(-1, keepdims=True)))[..., 0]
        tgt = np.take_along_axis(lg, batch[:, 1:, None], -1)[..., 0]
        tot += float((lse - tgt).sum())
        cnt += lse.size
    return float(np.exp(tot / cnt))
