"""Restructured fp32 stack with folded norms (src/turbo_roformer/fast.py) - test oracle.

The token layout stays (chunk, frame, band) for the whole stack and the axial grouping is a view, as in
``FastBSRoformer._transformer_torch`` (fast.py:222-266).  Folding follows ``_prep`` (fast.py:163-191):
``16 * gamma`` into the next Linear's input columns, the attention scale 1/8 into W_q, so every runtime
norm is x / max(|x|, 1e-12).
"""

from __future__ import annotations

from collections.abc import Mapping

import torch
import torch.nn.functional as F

from . import reference

Tensor = torch.Tensor
H, DH, DIM = 8, 64, 256


def fold(sd: Mapping[str, Tensor], depth: int) -> list[dict]:
    """Folded fp32 weights of the 2*depth sub-layers, block i time (mode 0) then freq (mode 1) (fast.py:127-134)."""
    out = []
    for i in range(depth):
        for mode in (0, 1):
            p = f"layers.{i}.{mode}.layers.0"
            ga = sd[f"{p}.0.norm.gamma"].float() * DIM**0.5
            wqkv = sd[f"{p}.0.to_qkv.weight"].float() * ga[None, :]
            wqkv[: H * DH] = wqkv[: H * DH] * 0.125
            wg = sd[f"{p}.0.to_gates.weight"].float() * ga[None, :]
            gf = sd[f"{p}.1.net.0.gamma"].float() * DIM**0.5
            out.append(
                dict(
                    mode=mode,
                    W=torch.cat([wqkv, wg]),
                    b=torch.cat([torch.zeros(3 * H * DH), sd[f"{p}.0.to_gates.bias"].float()]),
                    Wo=sd[f"{p}.0.to_out.0.weight"].float(),
                    W1=sd[f"{p}.1.net.1.weight"].float() * gf[None, :],
                    b1=sd[f"{p}.1.net.1.bias"].float(),
                    W2=sd[f"{p}.1.net.4.weight"].float(),
                    b2=sd[f"{p}.1.net.4.bias"].float(),
                    freqs=sd[f"{p}.0.rotary_embed.freqs"].float(),
                )
            )
    return out


def l2n(X: Tensor) -> Tensor:
    return X / X.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def attn_sublayer(X: Tensor, P: dict, dtype=torch.float32) -> Tensor:
    """Attention output (not yet added) for X (b, T, F, 256) (fast.py:226-249)."""
    b, T, Fq, _ = X.shape
    xn = l2n(X).to(dtype)
    qkvg = F.linear(xn, P["W"].to(dtype), P["b"].to(dtype))
    qkv = qkvg[..., : 3 * H * DH].view(b, T, Fq, 3, H, DH)
    g = qkvg[..., 3 * H * DH :].float().sigmoid()  # (b, T, F, H)
    if P["mode"] == 0:
        qkv = qkv.permute(3, 0, 2, 4, 1, 5)  # (3, b, F, H, T, D)
        L = T
    else:
        qkv = qkv.permute(3, 0, 1, 4, 2, 5)  # (3, b, T, H, F, D)
        L = Fq
    ang = reference.rotary_angles(L, P["freqs"])
    q, k, v = reference.rotate(qkv[0], ang), reference.rotate(qkv[1], ang), qkv[2]
    o = reference.softmax_attention(q.float(), k.float(), v.float(), 1.0).to(dtype)
    o = o.permute(0, 3, 1, 2, 4) if P["mode"] == 0 else o.permute(0, 1, 3, 2, 4)  # (b, T, F, H, D)
    o = (o * g.unsqueeze(-1).to(o.dtype)).reshape(b, T, Fq, H * DH)
    return F.linear(o, P["Wo"].to(dtype)).float()


def ff_sublayer(X: Tensor, P: dict, dtype=torch.float32) -> Tensor:
    """Feed-forward output (not yet added) (fast.py:251-257), exact-erf GELU."""
    xn = l2n(X).to(dtype)
    h = reference.gelu_erf(F.linear(xn, P["W1"].to(dtype), P["b1"].to(dtype)).float()).to(dtype)
    return F.linear(h, P["W2"].to(dtype), P["b2"].to(dtype)).float()


def attn_sublayer_sdpa(X: Tensor, P: dict, dtype=torch.bfloat16) -> Tensor:
    """``_attn_torch`` (fast.py:229-249) as the reference runs it in bf16: GEMMs in ``dtype``, rotary in fp32
    rounded back to ``dtype``, attention by ``F.scaled_dot_product_attention`` in ``dtype`` (scale 1, the
    1/8 is in W_q)."""
    b, T, Fq, _ = X.shape
    xn = l2n(X).to(dtype)
    qkvg = F.linear(xn, P["W"].to(dtype), P["b"].to(dtype))
    qkv = qkvg[..., : 3 * H * DH].view(b, T, Fq, 3, H, DH)
    g = qkvg[..., 3 * H * DH :].float().sigmoid()
    if P["mode"] == 0:
        qkv = qkv.permute(3, 0, 2, 4, 1, 5)
        L = T
    else:
        qkv = qkv.permute(3, 0, 1, 4, 2, 5)
        L = Fq
    ang = reference.rotary_angles(L, P["freqs"])
    q, k = reference.rotate(qkv[0], ang), reference.rotate(qkv[1], ang)
    o = F.scaled_dot_product_attention(q, k, qkv[2], scale=1.0)
    o = o.permute(0, 3, 1, 2, 4) if P["mode"] == 0 else o.permute(0, 1, 3, 2, 4)
    o = (o * g.unsqueeze(-1).to(o.dtype)).reshape(b, T, Fq, H * DH)
    return F.linear(o, P["Wo"].to(dtype)).float()


@torch.no_grad()
def stack_bf16_sdpa(X: Tensor, layers: list[dict]) -> Tensor:
    """The reference's portable bf16 path (``FastBSRoformer(dtype=bf16, glue="torch", attn="sdpa")``,
    fast.py:222-266): bf16 GEMMs (oneDNN on the CPU), bf16 SDPA, fp32 residual.  Used as a CPU timing
    baseline, not as a checker."""
    X = X.float().clone()
    for P in layers:
        X = X + attn_sublayer_sdpa(X, P)
        X = X + ff_sublayer(X, P, torch.bfloat16)
    return X


@torch.no_grad()
def stack(X: Tensor, layers: list[dict], dtype=torch.float32) -> Tensor:
    """``_transformer_torch`` (fast.py:259-266) on X (b, T, F, 256) fp32; returns a new tensor."""
    X = X.float().clone()
    for P in layers:
        X = X + attn_sublayer(X, P, dtype)
        X = X + ff_sublayer(X, P, dtype)
    return X


@torch.no_grad()
def mask(X: Tensor, sd: Mapping[str, Tensor], cfg) -> Tensor:
    """final norm + grouped band MLPs on the stack output (fast.py:349-360, 386-387) -> (b, T, mask width)."""
    return reference.mask_from_stack(X, sd, cfg)
