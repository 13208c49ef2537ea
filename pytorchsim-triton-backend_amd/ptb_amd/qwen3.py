"""Qwen3-8B decoder layer (prefill) composed from the HIP kernels.

The launch sequence is the reference bundle's: validation/pytorchsim/qwen3_8b_layer_prefill_2048x2048_bf16/
manifest.json lists 14 launches of 12 kernels, 00,01,02,03,04,03,05,06,07,08,00,09,10,11, and
:meth:`Qwen3Layer.forward` computes them in that order on the current HIP stream:

  K00 rmsnorm(x, w_in)            K01 q = xn Wq          K02 q-norm + RoPE -> [32,T,128]
  K03 k = xn Wk                   K04 k-norm + RoPE      K03 v = xn Wv      K05 v -> [8,T,128]
  K06 causal GQA attention        K07 o -> [T,32,128]    K08 h = o Wo + x
  K00 rmsnorm(h, w_post)          K09 gu = hn Wgu        K10 a = silu(g) * u
  K11 y = a Wd + h

K01 and the two K03 launches run as one GEMM over the concatenated weight [hidden, q|k|v] (one round
of 256x256 tiles fills the chip; the separate k and v GEMMs have 128 tiles each and leave half the
CUs idle), and K02, K04 and K05 read their column slices of its [T, q|k|v] output in place (the
same per-element arithmetic as the separate products).  K09 and K10 run as one kernel (``ops.gemm_swiglu``: the gate_up GEMM with silu(g) * u in its
epilogue, bit for bit the pair's result), so the [T, 2*I] gate_up product never goes to HBM, and
K06 writes O token-major, [T, 32, 128], so K07's transpose is not launched.

(The data flow is read from each kernel's index arithmetic; the reference times these kernels
separately and never runs the layer end to end, validation/gemm/simulate_shapes.py:279-302.)
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ops

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Qwen3Config:
    hidden: int = 4096
    intermediate: int = 12288
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    rope_theta: float = 1.0e6
    eps: float = 1e-6


QWEN3_8B = Qwen3Config()

LAUNCH_ORDER = ("00", "01", "02", "03", "04", "03", "05", "06", "07", "08", "00", "09", "10", "11")


def rope_tables(tokens: int, head_dim: int = 128, theta: float = 1.0e6, device="cpu"):
    """cos/sin [T, D] fp32 for rotate-half RoPE (angle t / theta^(2i/D), both halves alike),
    computed in fp64 on the host once per sequence length, like the model's cached tables."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    ang = torch.arange(tokens, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().float().to(device), emb.sin().float().to(device)


def random_weights(cfg: Qwen3Config = QWEN3_8B, seed: int = 0, std: float = 0.02, norm_mean: float = 1.0,
                   device="cpu") -> dict:
    """Random-init bf16 weights: projections ~N(0, std); the RMSNorm weights ~N(norm_mean, std)
    (norm_mean=1 keeps activations O(1) through the layer).  Drawn in a fixed order from one
    seeded generator.  Wgu is [hidden, 2*intermediate] = gate | up."""
    g = torch.Generator().manual_seed(seed)
    h, i, hd = cfg.hidden, cfg.intermediate, cfg.head_dim

    def draw(*shape, mean=0.0):
        return (torch.randn(*shape, generator=g) * std + mean).to(BF16).to(device)

    return {
        "w_in": draw(h, mean=norm_mean),
        "wq": draw(h, cfg.heads * hd),
        "wk": draw(h, cfg.kv_heads * hd),
        "wv": draw(h, cfg.kv_heads * hd),
        "w_qn": draw(hd, mean=norm_mean),
        "w_kn": draw(hd, mean=norm_mean),
        "wo": draw(cfg.heads * hd, h),
        "w_post": draw(h, mean=norm_mean),
        "wgu": draw(h, 2 * i),
        "wd": draw(i, h),
    }


class Qwen3Layer:
    """One decoder layer on the GPU; weights are device bf16 tensors as from :func:`random_weights`."""

    def __init__(self, weights: dict, cfg: Qwen3Config = QWEN3_8B):
        self.w = weights
        self.cfg = cfg
        self._tables = {}
        self._bufs = {}
        # the q, k and v projections run as one GEMM over [hidden, q|k|v] (a copy made once): one
        # round of 256x256 tiles on the chip instead of three GEMMs whose k and v parts leave most
        # CUs idle
        self.wqkv = torch.cat([weights["wq"], weights["wk"], weights["wv"]], dim=1).contiguous()

    def tables(self, tokens: int, device):
        key = (tokens, str(device))
        if key not in self._tables:
            self._tables[key] = rope_tables(tokens, self.cfg.head_dim, self.cfg.rope_theta, device)
        return self._tables[key]

    def buffers(self, tokens: int, device) -> dict:
        """Activation buffers for one forward at this length, allocated once and reused."""
        key = (tokens, str(device))
        if key not in self._bufs:
            c = self.cfg
            qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim

            def e(*shape):
                return torch.empty(*shape, dtype=BF16, device=device)

            self._bufs[key] = {
                "xn": e(tokens, c.hidden), "qkv": e(tokens, qd + 2 * kd),
                "kh": e(c.kv_heads, tokens, c.head_dim),
                "o": e(tokens, c.heads, c.head_dim), "h": e(tokens, c.hidden), "hn": e(tokens, c.hidden),
                "a": e(tokens, c.intermediate), "y": e(tokens, c.hidden),
            }
        return self._bufs[key]

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        c, w = self.cfg, self.w
        t = x.shape[0]
        cos, sin = self.tables(t, x.device)
        b = self.buffers(t, x.device)
        y = b["y"] if out is None else out
        ops.rmsnorm(x, w["w_in"], c.eps, out=b["xn"])                                       # K00
        qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim
        qkv = b["qkv"]
        ops.gemm(b["xn"], self.wqkv, out=qkv)                                              # K01 + K03
        # the k-norm reads its column slice of [T, q|k|v] in place; attention reads q (normalising and
        # rotating it in its prologue) and v there too, and writes O token-major
        ops.qk_norm_rope(qkv[:, qd:qd + kd].view(t, c.kv_heads, c.head_dim), w["w_kn"], cos, sin, c.eps,
                         out=b["kh"])                                                        # K04
        ops.flash_attention_qkv(qkv, b["kh"], w["w_qn"], cos, sin, c.heads, c.kv_heads, c.eps, True,
                                1.0 / math.sqrt(c.head_dim),
                                out=b["o"].view(1, t, c.heads, c.head_dim))                  # K02 K05 K06 K07
        ops.gemm(b["o"].view(t, c.heads * c.head_dim), w["wo"], residual=x, out=b["h"])     # K08
        ops.rmsnorm(b["h"], w["w_post"], c.eps, out=b["hn"])                                # K00
        ops.gemm_swiglu(b["hn"], w["wgu"], out=b["a"])                                      # K09 + K10
        ops.gemm(b["a"], w["wd"], residual=b["h"], out=y)                                   # K11
        return y

    __call__ = forward


# kernels Qwen3Layer.forward issues for the reference's 14 launches (K01 + K03 as one GEMM, K02 + K05
# + K06 + K07 in the attention kernel, K09 + K10 as one GEMM)
PREFILL_KERNELS = 8


class Qwen3DecodeLayer:
    """One decoder layer for a single new token over a KV cache, as the reference's decode bundle
    composes it (validation/pytorchsim/qwen3_8b_layer_decode_1x<S>_bf16/manifest.json, 8 launches):

      K00 ss = sum x^2                       K01 q = (x*r*w_in) Wq            (GEMV, fp32 prologue)
      K02 q-norm + RoPE (one position)       K03 decode attention over [8, S, 128] K/V
      K04 a = o Wo                           K05 ss2 = sum (x + a)^2
      K06 gu = ((x + a)*r2*w_post) Wgu       K07 y = (silu(g)*u) Wd + (x + a)

    (The bundle's decode layer reads the cache as given; it computes no k/v for the new token.)
    Issued as 9 kernels: each GEMV is a partial pass plus a finish pass, except that K06's finish
    runs inside K07's prologue, and attention is a partial pass plus a merge.
    Weights as from :func:`random_weights`; the GEMV and attention workspaces are allocated once."""

    def __init__(self, weights: dict, cfg: Qwen3Config = QWEN3_8B):
        self.w = weights
        self.cfg = cfg
        self._bufs = {}

    def buffers(self, seq: int, device) -> dict:
        key = (seq, str(device))
        if key not in self._bufs:
            c = self.cfg
            lib = ops._lib.load()
            gemv_ws = max(lib.ptb_gemv_workspace_bytes(c.hidden, c.heads * c.head_dim),
                          lib.ptb_gemv_workspace_bytes(c.heads * c.head_dim, c.hidden),
                          lib.ptb_gemv_workspace_bytes(c.hidden, 2 * c.intermediate),
                          lib.ptb_gemv_workspace_bytes(c.intermediate, c.hidden))
            attn_ws = lib.ptb_attn_decode_workspace_bytes(c.kv_heads, c.heads // c.kv_heads, seq)
            gu_parts = lib.ptb_gemv_workspace_bytes(c.hidden, 2 * c.intermediate)

            def e(*shape, dtype=BF16):
                return torch.empty(*shape, dtype=dtype, device=device)

            self._bufs[key] = {
                "ss": e(1, dtype=torch.float32), "q": e(c.heads * c.head_dim),
                "o": e(c.kv_heads, c.heads // c.kv_heads, c.head_dim), "a": e(c.hidden),
                "ss2": e(1, dtype=torch.float32), "y": e(c.hidden),
                "ws": e(max(gemv_ws, 4), dtype=torch.uint8), "attn_ws": e(max(attn_ws, 4), dtype=torch.uint8),
                "gu_parts": e(max(gu_parts, 4), dtype=torch.uint8),
            }
        return self._bufs[key]

    def forward(self, x: torch.Tensor, kcache: torch.Tensor, vcache: torch.Tensor, cos: torch.Tensor,
                sin: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """x [hidden] bf16; kcache/vcache [kv_heads, S, head_dim] bf16; cos/sin [head_dim] fp32 of the
        token's position."""
        c, w = self.cfg, self.w
        b = self.buffers(kcache.shape[1], x.device)
        y = b["y"] if out is None else out
        # K00's sum of squares is formed inside K01's (and K05's inside K06's) workgroups
        ops.gemv_rmsnorm(x, None, w["w_in"], w["wq"], eps=c.eps, out=b["q"], workspace=b["ws"])  # K00 + K01
        # K02's q-norm + RoPE runs in K03's prologue: each attention workgroup rotates its own q rows
        ops.attention_decode(b["q"].view(c.kv_heads, c.heads // c.kv_heads, c.head_dim), kcache, vcache,
                             1.0 / math.sqrt(c.head_dim), out=b["o"], workspace=b["attn_ws"],
                             qnorm=(w["w_qn"], cos, sin, c.eps))                                 # K02 + K03
        ops.gemv(b["o"].view(-1), w["wo"], out=b["a"], workspace=b["ws"])                      # K04
        # K05 + K06's partial pass; K06's finish runs in K07's prologue (the same sums and rounding)
        ops.gemv_rmsnorm_parts(x, None, w["w_post"], w["wgu"], add=b["a"], eps=c.eps, parts=b["gu_parts"])
        ops.gemv_silu_parts(b["gu_parts"], c.hidden, w["wd"], x, b["a"], out=y, workspace=b["ws"])  # K06 + K07
        return y

    __call__ = forward


def layer_work(tokens: int, cfg: Qwen3Config = QWEN3_8B) -> list:
    """(name, flops, hbm bytes) of each launch at this length: the roofline model of the layer
    (flop conventions as the reference reports: 2*M*N*K per GEMM, 4*H*D*S(S+1)/2 causal attention;
    bytes = each operand read once plus each output written once)."""
    c = cfg
    t, hd, i = tokens, c.hidden, c.intermediate
    qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim

    def mm(m, k, n, resid=False):
        return 2.0 * m * n * k, 2.0 * (m * k + k * n + m * n + (m * n if resid else 0))

    work = [("K00 rmsnorm", 4.0 * t * hd, 2.0 * (2 * t * hd + hd))]
    work.append(("K01 q_proj",) + mm(t, hd, qd))
    work.append(("K02 q_norm_rope", 10.0 * t * qd, 2.0 * 2 * t * qd + 8.0 * t * c.head_dim))
    work.append(("K03 k_proj",) + mm(t, hd, kd))
    work.append(("K04 k_norm_rope", 10.0 * t * kd, 2.0 * 2 * t * kd + 8.0 * t * c.head_dim))
    work.append(("K03 v_proj",) + mm(t, hd, kd))
    work.append(("K05 v_transpose", 0.0, 2.0 * 2 * t * kd))
    work.append(("K06 attention", 4.0 * c.heads * c.head_dim * t * (t + 1) / 2, 2.0 * (2 * t * qd + 2 * t * kd)))
    work.append(("K07 o_transpose", 0.0, 2.0 * 2 * t * qd))
    work.append(("K08 o_proj+res",) + mm(t, qd, hd, True))
    work.append(("K00 rmsnorm", 4.0 * t * hd, 2.0 * (2 * t * hd + hd)))
    work.append(("K09 gate_up",) + mm(t, hd, 2 * i))
    work.append(("K10 silu_mul", 5.0 * t * i, 2.0 * 3 * t * i))
    work.append(("K11 down+res",) + mm(t, i, hd, True))
    return work
