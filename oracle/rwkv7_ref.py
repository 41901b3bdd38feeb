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

Pinned by tests/test_oracle_forward.py with properties that do not retype
the formulas: token-by-token == whole-sequence, the w = 1, a = b = 0 case
equals the closed-form linear-attention sum, the decay identity
exp(-exp(-softplus(-z) - 0.5)) == exp(-0.606531 sigmoid(z)), and a
brute-force per-element recurrence on a tiny head.
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
            gate = _sigmoid(xv @ g("v1").T @ g("v2").T + g("v0").reshape(C))
            v = v + (v_first - v) * gate
        a = _sigmoid(xa @ g("a1").T @ g("a2").T + g("a0").reshape(C))
        gg = _sigmoid(xg @ g("g1").T) @ g("g2").T
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
        out = group_norm(y.reshape(B, T, C), H, g("ln_x.weight"),
                         g("ln_x.bias"))
        bonus = ((r.reshape(sh) * k.reshape(sh) * g("r_k").reshape(H, N))
                 .sum(-1, keepdims=True) * v.reshape(sh)).reshape(B, T, C)
        out = (out + bonus) * gg
        return out @ g("output.weight").T, v_first, (new_state, new_prev)

    def _cmix(self, i, x, prev):
        g = lambda s: self._g(f"blocks.{i}.ffn.{s}")
        sx, new_prev = self._shift(x, prev)
        xk = x + (sx - x) * g("x_k").reshape(-1)
        h = np.maximum(xk @ g("key.weight").T, 0.0) ** 2
        return h @ g("value.weight").T, new_prev

    def forward_stateful(self, idx, states, hidden_only=False):
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
        x = layer_norm(x, self._g("ln_out.weight"), self._g("ln_out.bias"))
        if hidden_only:
            return x, new_states
        return x @ self._g("head.weight").T, new_states
