"""Single sub-layers at the full 17 s chunk shape (62 bands x 1701 frames x 256): the time-attention,
frequency-attention and feed-forward blocks on N(0, 1) activations with N(0, 0.02) weights.

The device runs the whole shape; the oracle checks a subset that is independent of the rest: a few
bands for time attention (each band is its own sequence), a few frames for frequency attention, a few
thousand tokens for the feed-forward.  Each block's update (out - x) is compared with the fp32 forward
semantics (oracle.reference) and with the emulation of the same arithmetic (oracle.kernels).
"""

from __future__ import annotations

import pytest
import torch

from oracle import folded, kernels as ok, reference
from turbo_roformer_amd import weights
from turbo_roformer_amd.stack import HipStack

from .conftest import snr_db

pytestmark = pytest.mark.gpu
DEV = "cuda"
T, F = 1701, 62
CFG = dict(weights.RESURRECTION_CFG, depth=1)


@pytest.fixture(scope="module")
def sd():
    return weights.init_state_dict(CFG, seed=21, init="normal")


@pytest.fixture(scope="module")
def x_bf16():
    """x bf16 [frames, bands, 256] ~ N(0, 1), seeded."""
    g = torch.Generator().manual_seed(22)
    return torch.randn(T, F, 256, generator=g).to(torch.bfloat16)


@pytest.fixture(scope="module", params=["ff_fp16", "ff_split", "bf16"])
def stack(request, hip, sd):
    return HipStack(sd, DEV, precision=request.param)


def _run(stack, x, fn, layer):
    X = x.float().reshape(-1, 256).contiguous().to(DEV)
    fn(X, 1, T, F, layer)
    torch.cuda.synchronize()
    return X.cpu().view(T, F, 256)


def _emulate_attn(P, xs, mode):
    """The bf16 kernel sequence of one attention sub-layer on tokens xs [T', F', 256] (oracle)."""
    Tq, Fq = xs.shape[0], xs.shape[1]
    X = xs.reshape(-1, 256).float()
    w = ok.bf16_weights(P)
    _, xn = ok.add_rmsnorm(X, None)
    Q, K, Vt, G = ok.qkv_rope(xn, w["W"], w["b_gate"], w["freqs"], mode, 1, Tq, Fq)
    O = ok.attention(Q, K, Vt, G, mode, 1, Tq, Fq)
    y, _ = ok.gemm_res_norm(O, w["Wo"], None, X)
    return y.view(Tq, Fq, 256)


@pytest.mark.parametrize("mode", [0, 1])
def test_attention_block_full_shape(stack, sd, x_bf16, mode):
    """Config 2 (mode 0: 62 x 8 sequences of 1701 frames) and config 3 (mode 1: 1701 x 8 sequences of
    62 bands).  The out-projection is bf16 in both precisions, so the emulation is the same."""
    print(f"attn block full shape mode={mode} precision={stack.precision}", flush=True)
    out = _run(stack, x_bf16, stack.attn_block, mode)
    x = x_bf16.float()
    assert torch.isfinite(out).all()
    prefix = f"layers.0.{mode}.layers.0.0"
    P = folded.fold(sd, 1)[mode]
    if mode == 0:
        sel = torch.tensor([0, 17, 40, 61])
        xs = x[:, sel]  # [T, 4, 256]: 4 complete band sequences
        ref = reference.attention(xs.transpose(0, 1).double(), {k: v.double() for k, v in sd.items()}, prefix)
        ref = ref.transpose(0, 1).float()
        got = out[:, sel] - xs
    else:
        sel = torch.tensor([0, 1, 850, 1699, 1700])
        xs = x[sel]  # [5, F, 256]: 5 complete frame sequences
        ref = reference.attention(xs.double(), {k: v.double() for k, v in sd.items()}, prefix).float()
        got = out[sel] - xs
    emu = _emulate_attn(P, xs, mode) - xs
    s_ref, s_emu = snr_db(ref.numpy(), got.numpy()), snr_db(emu.numpy(), got.numpy())
    s_design = snr_db(ref.numpy(), emu.numpy())
    print(f"  update snr vs fp32 {s_ref:.1f} dB (bf16 design {s_design:.1f} dB), vs emulation {s_emu:.1f} dB")
    assert s_emu >= 45.0
    assert s_ref >= s_design - 1.0
    # absolute floor against the fp32 forward (the bf16 design measures 47.6-47.8 dB on this input), so a
    # drift of the emulation cannot move the bar with it
    assert s_ref >= 46.0


def test_feed_forward_block_full_shape(stack, sd, x_bf16):
    """Config 4: 105,462 tokens x 256 through norm, FF1 + GELU, FF2 + residual."""
    print(f"ff block full shape precision={stack.precision}", flush=True)
    out = _run(stack, x_bf16, stack.ff_block, 0)
    x = x_bf16.float().reshape(-1, 256)
    out = out.reshape(-1, 256)
    assert torch.isfinite(out).all()
    sel = torch.randperm(T * F, generator=torch.Generator().manual_seed(23))[:4096]
    xs = x[sel]
    prefix = "layers.0.0.layers.0.1"
    ref = reference.feed_forward(xs.double(), {k: v.double() for k, v in sd.items()}, prefix).float()
    P = folded.fold(sd, 1)[0]
    if stack.precision == "ff_split":
        y, _ = ok.ff_split(xs, P["W1"], P["b1"], P["W2"], P["b2"])
    elif stack.precision == "ff_fp16":
        y, _ = ok.ff_fp16(xs, P["W1"], P["b1"], P["W2"], P["b2"])
    else:
        w = ok.bf16_weights(P)
        _, xn = ok.add_rmsnorm(xs, None)
        y, _ = ok.gemm_res_norm(ok.gemm_gelu(xn, w["W1"], w["b1"]), w["W2"], w["b2"], xs)
    emu = y - xs
    got = out[sel] - xs
    s_ref, s_emu, s_design = snr_db(ref.numpy(), got.numpy()), snr_db(emu.numpy(), got.numpy()), snr_db(ref.numpy(), emu.numpy())
    print(f"  update snr vs fp32 {s_ref:.1f} dB (design {s_design:.1f} dB), vs emulation {s_emu:.1f} dB")
    if stack.precision == "ff_split":
        # split operands: ~2^-16 relative products; the remaining error is the fp32 GELU (A&S 7.1.26)
        assert s_ref >= 90.0
    elif stack.precision == "ff_fp16":
        assert s_ref >= s_design - 1.0 and s_design >= 65.0  # fp16 operands: ~18 dB above bf16
        assert s_ref >= 66.0  # absolute floor (68.3 dB measured)
    else:
        assert s_ref >= s_design - 1.0
        assert s_ref >= 48.5  # absolute floor (50.2 dB measured)
    assert s_emu >= 50.0
