"""bf16-rounding emulations of the reference's fused CPU ops, on the device layouts - test oracle.

Each function reproduces where the reference kernels (src/turbo_roformer/csrc/kernels.cpp) round to
bf16 and what they keep in fp32, with fp64 accumulation, so that a correct device kernel differs from
it only by fp32 summation order (occasionally one bf16 step at a rounding boundary).  Inputs and outputs
use the sequence-buffer layouts of include/trf_hip.h: Q, K chunk-major [nseq, 8, 8, Lpad, 8], Vt [nseq, 8, 64, Lpad]
bf16, G [ntok, 8] fp32, tokens in (chunk, frame, band) order.
"""

from __future__ import annotations

import math

import torch

from . import reference

Tensor = torch.Tensor
H, DH, DIM, HID = 8, 64, 256, 1024
LOG2E = 1.44269504088896341


def seq_pad(L: int) -> int:
    return (L + 63) // 64 * 64


def token_index(mode: int, batch: int, T: int, F: int) -> Tensor:
    """[nseq, L] token of position p in sequence s: time s=(c, f), p=t; freq s=(c, t), p=f (kernels.cpp:201)."""
    tok = torch.arange(batch * T * F).view(batch, T, F)
    if mode == 0:
        return tok.permute(0, 2, 1).reshape(batch * F, T)
    return tok.reshape(batch * T, F)


def l2_rows(X: Tensor) -> Tensor:
    return X / X.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def add_rmsnorm(X: Tensor, Y: Tensor | None, out_dtype=torch.bfloat16) -> tuple[Tensor, Tensor]:
    """add_rmsnorm (kernels.cpp:101-137): X' = X + Y; out = X' / max(|X'|, 1e-12)."""
    Xn = X.float() + (Y.float() if Y is not None else 0.0)
    out = (Xn.double() / Xn.double().norm(dim=-1, keepdim=True).clamp_min(1e-12)).to(out_dtype)
    return Xn, out


def qk_chunk_major(X: Tensor) -> Tensor:
    """[nseq, H, Lpad, 64] -> the device's chunk-major [nseq, H, 8, Lpad, 8] (trf_hip.h)."""
    nseq, h, lp, d = X.shape
    return X.view(nseq, h, lp, d // 8, 8).permute(0, 1, 3, 2, 4).contiguous()


def qk_rows(X: Tensor) -> Tensor:
    """Chunk-major [nseq, H, 8, Lpad, 8] -> rows [nseq, H, Lpad, 64]."""
    nseq, h, c, lp, e = X.shape
    return X.permute(0, 1, 3, 2, 4).reshape(nseq, h, lp, c * e)


def qkv_rope(xn: Tensor, W: Tensor, b_gate: Tensor, freqs: Tensor, mode: int, batch: int, T: int, F: int):
    """qkv_rope_gemm (kernels.cpp:439-540): fp32 accumulators, fp32 rotary of q and k, bf16 outputs,
    fp32 sigmoid gates.  Returns Q, K, Vt (padded, zero pads) and G.

    Device contract: q leaves multiplied by log2(e) (in fp32, before its single bf16 rounding), so that
    q.k is the base-2 exponent of the softmax; the reference multiplies by log2(e) inside its exp
    (kernels.cpp:333-339).  The two differ only in where q is rounded."""
    n = xn.shape[0]
    acc = (xn.double() @ W.double().t()).float()  # [n, 1544]
    g = torch.sigmoid(acc[:, 3 * H * DH :].double() + b_gate.double()).float()
    idx = token_index(mode, batch, T, F)
    nseq, L = idx.shape
    Lp = seq_pad(L)
    ang = reference.rotary_angles(L, freqs)  # [L, 32]

    def seq(part: int) -> Tensor:  # [nseq, H, L, DH] fp32
        x = acc[:, part * H * DH : (part + 1) * H * DH].view(n, H, DH)
        return x[idx].permute(0, 2, 1, 3)

    q = (reference.rotate(seq(0), ang) * torch.tensor(LOG2E, dtype=torch.float32)).to(torch.bfloat16)
    k = reference.rotate(seq(1), ang).to(torch.bfloat16)
    v = seq(2).to(torch.bfloat16)
    Q = torch.zeros(nseq, H, Lp, DH, dtype=torch.bfloat16)
    K = torch.zeros_like(Q)
    Vt = torch.zeros(nseq, H, DH, Lp, dtype=torch.bfloat16)
    Q[:, :, :L] = q
    K[:, :, :L] = k
    Vt[:, :, :, :L] = v.transpose(-1, -2)
    return qk_chunk_major(Q), qk_chunk_major(K), Vt, g


def attention(Q: Tensor, K: Tensor, Vt: Tensor, G: Tensor, mode: int, batch: int, T: int, F: int,
              chunk: int = 64, shift: str = "device") -> Tensor:
    """attention (kernels.cpp:250-388): exact row max m over valid keys, e = 2^(s - m) in fp32 (Q carries
    log2(e), see qkv_rope), unnormalised bf16 P, fp32 row sum of e, O = (P V) * gate / sum rounded to
    bf16, token order.

    ``shift="max"`` is the reference's shift m.  ``shift="device"`` follows the library: sequences of more
    than 64 positions go through the single-sweep kernel, whose shift is an integer >= m and whose
    normaliser is the sum of the rounded P instead of e; with an integer shift P = 2^-c bf16(2^s), so
    every integer gives the same result and ceil(m) stands for it here.  Sequences of up to 64 positions
    keep m and the sum of e."""
    if shift not in ("device", "max"):
        raise ValueError("shift must be 'device' or 'max'")
    idx = token_index(mode, batch, T, F)
    nseq, L = idx.shape
    Q, K = qk_rows(Q), qk_rows(K)
    O = torch.empty(batch * T * F, H * DH, dtype=torch.bfloat16)
    for s0 in range(0, nseq, chunk):
        s1 = min(nseq, s0 + chunk)
        q = Q[s0:s1, :, :L].double()
        k = K[s0:s1, :, :L].double()
        v = Vt[s0:s1, :, :, :L].double().transpose(-1, -2)
        S = (q @ k.transpose(-1, -2)).float()
        m = S.amax(dim=-1, keepdim=True)
        single_sweep = shift == "device" and L > 64
        if single_sweep:
            m = torch.ceil(m)
        e = torch.exp2(S - m)  # fp32
        P = e.to(torch.bfloat16).double()
        rs = (P if single_sweep else e.double()).sum(dim=-1, keepdim=True)
        o = P @ v  # [s, H, L, DH]
        tok = idx[s0:s1]  # [s, L]
        gate = G[tok].permute(0, 2, 1).unsqueeze(-1).double()  # [s, H, L, 1]
        o = (o * (gate / rs)).to(torch.bfloat16)
        O.view(-1, H, DH)[tok] = o.permute(0, 2, 1, 3)
    return O


def gemm_res_norm(A: Tensor, W: Tensor, bias: Tensor | None, X: Tensor) -> tuple[Tensor, Tensor]:
    """gemm_res_norm (kernels.cpp:542-586): X' = X + A W^T (+ b) in fp32; xn = X'/|X'| as bf16."""
    y = (A.double() @ W.double().t()).float() + X.float()
    if bias is not None:
        y = y + bias.float()
    xn = (y.double() / y.double().norm(dim=-1, keepdim=True).clamp_min(1e-12)).to(torch.bfloat16)
    return y, xn


def gemm_gelu(xn: Tensor, W1: Tensor, b1: Tensor) -> Tensor:
    """gemm_gelu (kernels.cpp:609-642) with the exact erf: H = gelu(xn W1^T + b1) as bf16."""
    x = (xn.double() @ W1.double().t()).float() + b1.float()
    return (0.5 * x.double() * (1.0 + torch.erf(x.double() / math.sqrt(2.0)))).to(torch.bfloat16)


def split_bf16(x: Tensor) -> tuple[Tensor, Tensor]:
    """Split-bf16 parts of fp32 x: hi = bf16(x), lo = bf16(x - hi)."""
    x = x.float()
    hi = x.to(torch.bfloat16)
    return hi, (x - hi.float()).to(torch.bfloat16)


def split_matmul(a: Tensor, w_hi: Tensor, w_lo: Tensor) -> Tensor:
    """a W^T from split-bf16 operands: hi.hi + lo.hi + hi.lo (the lo.lo term dropped), fp64 sums, fp32 out."""
    ah, al = split_bf16(a)
    wh, wl = w_hi.double().t(), w_lo.double().t()
    return (ah.double() @ wh + al.double() @ wh + ah.double() @ wl).float()


def ff_split(X: Tensor, W1: Tensor, b1: Tensor, W2: Tensor, b2: Tensor) -> tuple[Tensor, Tensor]:
    """The feed-forward sub-layer in the library's split precision (TRF_PREC_FF_SPLIT): xn = X/|X| in
    fp32, both GEMMs on split-bf16 operands of xn, W1, gelu(h), W2 (fp32 weights split here); returns the
    fp32 residual stream and the bf16 xn of the result.  Not a reference kernel: this is the library's
    own higher-precision mode, checked against the fp32 forward."""
    xn = (X.double() / X.double().norm(dim=-1, keepdim=True).clamp_min(1e-12)).float()
    h = split_matmul(xn, *split_bf16(W1)) + b1.float()
    g = (0.5 * h.double() * (1.0 + torch.erf(h.double() / math.sqrt(2.0)))).float()
    y = X.float() + split_matmul(g, *split_bf16(W2)) + b2.float()
    return y, (y.double() / y.double().norm(dim=-1, keepdim=True).clamp_min(1e-12)).to(torch.bfloat16)


def ff_fp16(X: Tensor, W1: Tensor, b1: Tensor, W2: Tensor, b2: Tensor) -> tuple[Tensor, Tensor]:
    """The feed-forward sub-layer in the library's fp16 precision (TRF_PREC_FF_FP16): xn = X/|X| in fp32,
    then xn, W1, gelu(h) and W2 rounded to fp16 (round to nearest even) with fp64 sums here; returns the
    fp32 residual stream and the bf16 xn of the result.  Not a reference kernel: the library's own mode."""
    xn = (X.double() / X.double().norm(dim=-1, keepdim=True).clamp_min(1e-12)).float()
    h = (xn.half().double() @ W1.float().half().double().t()).float() + b1.float()
    g = (0.5 * h.double() * (1.0 + torch.erf(h.double() / math.sqrt(2.0)))).float()
    y = X.float() + (g.half().double() @ W2.float().half().double().t()).float() + b2.float()
    return y, (y.double() / y.double().norm(dim=-1, keepdim=True).clamp_min(1e-12)).to(torch.bfloat16)


def bf16_weights(P: dict) -> dict:
    """bf16 operands of one folded sub-layer (oracle.folded.fold output), as the kernels see them."""
    return dict(
        mode=P["mode"], W=P["W"][: 3 * H * DH + H].to(torch.bfloat16), b_gate=P["b"][3 * H * DH :].float(),
        Wo=P["Wo"].to(torch.bfloat16), W1=P["W1"].to(torch.bfloat16), b1=P["b1"].float(),
        W2=P["W2"].to(torch.bfloat16), b2=P["b2"].float(), freqs=P["freqs"],
    )


@torch.no_grad()
def stack(X: Tensor, layers: list[dict], batch: int, T: int, F: int, precision: str = "bf16") -> Tensor:
    """The fused-op sequence of ``_transformer_cpp`` (fast.py:269-341) with bf16 rounding at the same
    points as the reference kernels; X is [batch*T*F, 256] fp32, returns a new tensor.
    ``precision="ff_split"`` / ``"ff_fp16"`` replaces the feed-forward by ``ff_split`` / ``ff_fp16``."""
    X = X.float().clone()
    _, xn = add_rmsnorm(X, None)
    for P in layers:
        w = bf16_weights(P)
        Q, K, Vt, G = qkv_rope(xn, w["W"], w["b_gate"], w["freqs"], w["mode"], batch, T, F)
        O = attention(Q, K, Vt, G, w["mode"], batch, T, F)
        X, xn = gemm_res_norm(O, w["Wo"], None, X)
        if precision in ("ff_split", "ff_fp16"):
            X, xn = (ff_split if precision == "ff_split" else ff_fp16)(X, P["W1"], P["b1"], P["W2"], P["b2"])
            continue
        Hh = gemm_gelu(xn, w["W1"], w["b1"])
        X, xn = gemm_res_norm(Hh, w["W2"], w["b2"], X)
    return X


def _split_f16(v: Tensor) -> tuple[Tensor, Tensor]:
    """v (fp32) -> fp16 hi = f16(v) and lo = f16(v - hi), both returned as float64."""
    v = v.float()
    hi = v.half()
    return hi.double(), (v - hi.float()).half().double()


def _mm_f16(a: Tensor, w: Tensor, split: bool) -> Tensor:
    """a @ w^T with fp16 operands and fp64 sums: hi.hi + hi.lo + lo.hi when split, else hi.hi."""
    ah, al = _split_f16(a)
    wh, wl = _split_f16(w)
    out = ah @ wh.t()
    if split:
        out = out + al @ wh.t() + ah @ wl.t()
    return out


@torch.no_grad()
def mask_head(x: Tensor, sd, dims: tuple[int, ...], precision: str = "split") -> Tensor:
    """Final RMSNorm + per-band mask MLP (fast.py:349-360, model.py:158-178) at the rounding points of the
    library's trf_mask_head: xn = x / max(|x|, 1e-12) * 16 in fp32, W1 * gamma folded in fp32, then xn,
    W1, tanh(h) and W2 rounded to fp16 hi (and lo = f16(v - hi) with ``precision="split"``), products
    hi.hi (+ hi.lo + lo.hi) summed in fp64, biases and GLU in fp64.  Not a reference kernel: the library's
    own arithmetic.  x: (..., bands, 256) -> (..., sum(dims))."""
    split = precision == "split"
    xf = x.float()
    xn = (xf / xf.norm(dim=-1, keepdim=True).clamp_min(1e-12)) * DIM**0.5
    g = sd["final_norm.gamma"].float()
    outs = []
    for i, d in enumerate(dims):
        p = f"mask_estimators.0.to_freqs.{i}.0"
        w1 = sd[f"{p}.0.weight"].float() * g[None, :]
        h = torch.tanh(_mm_f16(xn[..., i, :], w1, split) + sd[f"{p}.0.bias"].double())
        o = _mm_f16(h.float(), sd[f"{p}.2.weight"].float(), split) + sd[f"{p}.2.bias"].double()
        outs.append(o[..., :d] * torch.sigmoid(o[..., d:]))
    return torch.cat(outs, dim=-1)
