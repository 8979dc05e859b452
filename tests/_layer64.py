"""Float64 restatement of one quantized decoder layer on the GPU (torch), for condition-aware bounds.

Test infrastructure only: it never stands in for the HIP path.  It follows the structure of the
reference layer (hls/decode_only/qwen_decode_attention_kernel.cpp:13-162 and
qwen_decode_mlp_kernel.cpp:44-119 for decode; hls/prefill_only/qwen_prefill_attention_kernel.cpp:112-289
and qwen_prefill_mlp_kernel.cpp:217-332 for prefill): RMSNorm, Q/K/V projections with bias, RoPE on
pairs (p, p + 64), GQA attention (query head h reads KV head h // 6), the O projection with no input
residual, RMSNorm, SwiGLU gate/up, the down projection plus the attention output.  Everything is
evaluated in float64 with exact elementary functions (the decode reference's libm calls; the
prefill reference's approx_sqrt/approx_exp/approx_sincos differ from them by far less than the
bounds below need).

Besides the values it returns, for every output element, the absolute-value sum of the projection
that produces it: A_i = sum_j |x_j| |w_ij| (+ |bias_i|), the condition term of a dot product.  The
FAST path codes each activation row with about 15 bits (a step of max|x| / 32512), so its error per
output is a small multiple of 2^-15 A_i; a fixed fraction of max|y| cannot say that for the small
elements of a tensor.  For the layer output (a + down(s)) the term is A_down + A_o; for a rotated K
element it is the sum of the terms of its RoPE pair.
"""

from __future__ import annotations

import math

import numpy as np

from work_llm_accelerator_amd.layout import HEAD_DIM, HIDDEN, INTERMEDIATE, KV_WIDTH, LAYOUT, Q_HEADS
from work_llm_accelerator_amd.quant import layer_views

ROPE_THETA = 1.0e6
EPS = 1.0e-6


def _dequant(torch, packed: np.ndarray, scales: np.ndarray, out_dim: int, in_dim: int, dev):
    """INT4 nibbles (even flat index in the low nibble) times the per-row scale, float64 [out, in]."""
    p = torch.from_numpy(np.ascontiguousarray(packed)).to(dev)
    nib = torch.stack([p & 0xF, p >> 4], dim=1).reshape(out_dim, in_dim).to(torch.int16)
    q = torch.where(nib >= 8, nib - 16, nib).to(torch.float64)
    return q * torch.from_numpy(np.ascontiguousarray(scales)).to(dev).to(torch.float64)[:, None]


class Layer64:
    """Dequantized float64 parameters of one layer image, resident on the GPU."""

    def __init__(self, torch, weight_ddr: np.ndarray, scale_ddr: np.ndarray, device="cuda"):
        self.t = torch
        v = layer_views(weight_ddr, scale_ddr)
        f64 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device).to(torch.float64)  # noqa: E731
        self.wq = _dequant(torch, v["q_w"], v["q_s"], HIDDEN, HIDDEN, device)
        self.wk = _dequant(torch, v["k_w"], v["k_s"], KV_WIDTH, HIDDEN, device)
        self.wv = _dequant(torch, v["v_w"], v["v_s"], KV_WIDTH, HIDDEN, device)
        self.wo = _dequant(torch, v["o_w"], v["o_s"], HIDDEN, HIDDEN, device)
        self.wg = _dequant(torch, v["gate_w"], v["gate_s"], INTERMEDIATE, HIDDEN, device)
        self.wu = _dequant(torch, v["up_w"], v["up_s"], INTERMEDIATE, HIDDEN, device)
        self.wd = _dequant(torch, v["down_w"], v["down_s"], HIDDEN, INTERMEDIATE, device)
        self.bq, self.bk, self.bv = f64(v["q_bias"]), f64(v["k_bias"]), f64(v["v_bias"])
        self.ln, self.post_ln = f64(v["input_layernorm"]), f64(v["post_attention_layernorm"])
        self.abs = {n: getattr(self, n).abs() for n in ("wk", "wv", "wo", "wd")}

    @classmethod
    def from_model(cls, torch, model, layer: int):
        w = np.zeros(LAYOUT.total_parameter_bytes, np.uint8)
        s = np.zeros(LAYOUT.total_parameter_bytes // 4, np.float32)
        assert model.lib.qwen_hip_model_layer_images(model.handle, layer, w, s) == 0
        return cls(torch, w, s)

    # ---- pieces -----------------------------------------------------------------------------
    def _rms(self, x, w):
        return x / self.t.sqrt(self.t.mean(x * x, dim=-1, keepdim=True) + EPS) * w

    def _proj(self, x, name, bias=None, terms=True):
        """(x W^T + b, |x| |W|^T + |b| or None) over the last dimension of x."""
        y = x @ getattr(self, name).T
        a = x.abs() @ self.abs[name].T if terms else None
        if bias is not None:
            y = y + bias
            if terms:
                a = a + bias.abs()
        return y, a

    def _rope(self, m, pos, heads):
        """m [..., heads*128] rotated at positions pos [...] (float64 angles, theta = 1e6)."""
        t = self.t
        p = t.arange(64, device=m.device, dtype=t.float64)
        inv = t.pow(t.tensor(ROPE_THETA, dtype=t.float64, device=m.device), -2.0 * p / HEAD_DIM)
        ang = pos.to(t.float64)[..., None] * inv
        c, s = t.cos(ang)[..., None, :], t.sin(ang)[..., None, :]
        h = m.reshape(*m.shape[:-1], heads, HEAD_DIM)
        e, o = h[..., :64], h[..., 64:]
        return t.cat([e * c - o * s, o * c + e * s], dim=-1).reshape(m.shape)

    @staticmethod
    def _pair_terms(t, a, heads):
        """Condition term of a rotated element: the sum of its pair's terms (|cos|, |sin| <= 1)."""
        h = a.reshape(*a.shape[:-1], heads, HEAD_DIM)
        s = h[..., :64] + h[..., 64:]
        return t.cat([s, s], dim=-1).reshape(a.shape)

    def _mlp(self, a):
        """a [..., 1536] -> (out, A_out without the O term)."""
        t = self.t
        post = self._rms(a, self.post_ln)
        g, _ = self._proj(post, "wg", terms=False)
        u, _ = self._proj(post, "wu", terms=False)
        s = g / (1.0 + t.exp(-g)) * u
        dn, a_dn = self._proj(s, "wd")
        return a + dn, a_dn

    # ---- layers -----------------------------------------------------------------------------
    def decode(self, x, positions, k_hist, v_hist):
        """One decode step of B sequences.
        x [B,1536] float64; positions [B] (the new token's position p_b); k_hist / v_hist [B,T,256] fp32 or
        float64 holding rows 0..p_b-1 of each sequence (T >= max p_b + 1; rows at or past p_b are ignored).
        Returns a dict of float64 tensors: out, k, v (the new rows) and their terms a_out, a_k, a_v."""
        t = self.t
        B = x.shape[0]
        n = self._rms(x, self.ln)
        q, _ = self._proj(n, "wq", self.bq, terms=False)
        k, a_k = self._proj(n, "wk", self.bk)
        v, a_v = self._proj(n, "wv", self.bv)
        pos = positions.to(x.device).to(t.int64)
        q = self._rope(q, pos, Q_HEADS)
        k = self._rope(k, pos, 2)
        a_k = self._pair_terms(t, a_k, 2)
        T = int(pos.max().item()) + 1
        K = k_hist[:, :T].to(t.float64).clone()
        V = v_hist[:, :T].to(t.float64).clone()
        idx = t.arange(B, device=x.device)
        K[idx, pos] = k
        V[idx, pos] = v
        mask = t.arange(T, device=x.device)[None, :] <= pos[:, None]  # [B,T]
        qh = q.reshape(B, 2, Q_HEADS // 2, HEAD_DIM)
        Kh = K.reshape(B, T, 2, HEAD_DIM).permute(0, 2, 3, 1).contiguous()  # [B,2,128,T]
        Vh = V.reshape(B, T, 2, HEAD_DIM).permute(0, 2, 1, 3).contiguous()  # [B,2,T,128]
        sc = (qh @ Kh) / math.sqrt(HEAD_DIM)  # [B,2,6,T]
        sc = sc.masked_fill(~mask[:, None, None, :], float("-inf"))
        p = t.softmax(sc, dim=-1)
        ctx = (p @ Vh).reshape(B, HIDDEN)
        a, a_o = self._proj(ctx, "wo")
        out, a_dn = self._mlp(a)
        return {"out": out, "k": k, "v": v, "a_out": a_dn + a_o, "a_k": a_k, "a_v": a_v}

    def prefill(self, x):
        """Prefill of B sequences of S tokens at positions 0..S-1 (causal).  x [B,S,1536] float64.
        Returns out, k, v [B,S,...] and their terms as in decode."""
        t = self.t
        B, S, _ = x.shape
        n = self._rms(x, self.ln)
        q, _ = self._proj(n, "wq", self.bq, terms=False)
        k, a_k = self._proj(n, "wk", self.bk)
        v, a_v = self._proj(n, "wv", self.bv)
        pos = t.arange(S, device=x.device)[None, :].expand(B, S)
        q = self._rope(q, pos, Q_HEADS)
        k = self._rope(k, pos, 2)
        a_k = self._pair_terms(t, a_k, 2)
        ctx = t.empty(B, S, Q_HEADS, HEAD_DIM, dtype=t.float64, device=x.device)
        causal = t.ones(S, S, dtype=t.bool, device=x.device).tril()
        for b in range(B):
            for kv in range(2):
                Kt = k[b].reshape(S, 2, HEAD_DIM)[:, kv].T.contiguous()  # [128,S]
                Vb = v[b].reshape(S, 2, HEAD_DIM)[:, kv].contiguous()  # [S,128]
                qb = q[b].reshape(S, Q_HEADS, HEAD_DIM)[:, kv * 6:(kv + 1) * 6].permute(1, 0, 2)  # [6,S,128]
                sc = (qb @ Kt) / math.sqrt(HEAD_DIM)
                sc = sc.masked_fill(~causal, float("-inf"))
                ctx[b, :, kv * 6:(kv + 1) * 6] = (t.softmax(sc, dim=-1) @ Vb).permute(1, 0, 2)
        a, a_o = self._proj(ctx.reshape(B, S, HIDDEN), "wo")
        out, a_dn = self._mlp(a)
        return {"out": out, "k": k, "v": v, "a_out": a_dn + a_o, "a_k": a_k, "a_v": a_v}


def ratio_to_bound(torch, got, ref, term) -> float:
    """max_i |got_i - ref_i| / (2^-15 term_i): the constant c of the per-element bound that the
    tensor meets (float64)."""
    d = (got.to(torch.float64) - ref.to(torch.float64)).abs()
    return float((d / (term.to(torch.float64) * 2.0 ** -15)).max().item())


def rel_to_max(torch, got, ref) -> float:
    """max |got - ref| / max |ref| (float64)."""
    r = ref.to(torch.float64)
    return float(((got.to(torch.float64) - r).abs().max() / r.abs().max()).item())
