"""The fused QKV + rotary + gates + attention kernel for sequences of at most 64 positions
(``trf_qkv_attention_short``, used by the stack for frequency attention) against the oracle's emulation
of the reference's two ops (qkv_rope_gemm, then attention: kernels.cpp:439-540, 250-388), and against the
library's unfused pair on the same inputs.

Shapes: the 62-band frequency attention (batched, up to the 300-frame chunk), 64 and 33 positions, one
position, and time attention of chunks of at most 64 frames.  The q and k rows of the weights are scaled up so
that the scores span tens of units (peaked softmax rows).  Tolerance: the per-op bar of the unfused
kernels (two bf16 steps elementwise, one rounding flip in 1e-4 of the elements, SNR floor), and every
output token written.
"""

from __future__ import annotations

import pytest
import torch

from oracle import folded, kernels as ok
from turbo_roformer_amd import _hip, weights
from turbo_roformer_amd.stack import rope_table

from .conftest import assert_bf16_close, rand_x, snr_db

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [  # (mode, batch, T, F)
    (1, 1, 300, 62),
    (1, 2, 37, 62),
    (1, 3, 11, 64),
    (1, 1, 9, 33),
    (1, 1, 5, 1),
    (1, 1, 100, 7),
    (0, 1, 64, 3),
    (0, 1, 40, 5),
    (0, 2, 1, 5),
    # group and head splits between the kernel's workgroups (one per CU, an even share of
    # (4-sequence group, head) units each): 3 x 257 = 771 sequences (1,544 units), 2 x 129 = 258 (520)
    (1, 3, 257, 64),
    (1, 2, 129, 45),
]


@pytest.fixture(scope="module")
def sharp_layers(hip):
    """(bf16 weights, packed layer) of a time and a freq sub-layer with the q and k rows scaled by 6."""
    cfg = dict(weights.TINY_CFG, depth=1)
    sd = weights.init_state_dict(cfg, seed=5, init="normal")
    out = []
    for P in folded.fold(sd, 1):
        w = ok.bf16_weights(P)
        W = w["W"].float().clone()
        W[:1024] *= 6.0
        w["W"] = W.to(torch.bfloat16)
        packed = torch.empty(_hip.layer_packed_bytes(), dtype=torch.uint8, device=DEV)
        _hip.pack_layer(w["W"].to(DEV), w["b_gate"].to(DEV), w["Wo"].to(DEV), w["W1"].to(DEV), w["b1"].to(DEV),
                        w["W2"].to(DEV), w["b2"].to(DEV), out=packed)
        out.append((w, packed))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("mode,batch,T,F", SHAPES)
def test_fused_short_attention(sharp_layers, mode, batch, T, F):
    w, packed = sharp_layers[mode]
    n = batch * T * F
    L = T if mode == 0 else F
    xn = ok.l2_rows(rand_x(n, 40 + T + F)).to(torch.bfloat16)
    Q, K, Vt, G = ok.qkv_rope(xn, w["W"], w["b_gate"], w["freqs"], mode, batch, T, F)
    Oref = ok.attention(Q, K, Vt, G, mode, batch, T, F)
    xd = xn.to(DEV)
    rope = rope_table(w["freqs"], L).to(DEV)
    O = torch.full((n, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    print(f"fused short attention mode={mode} batch={batch} T={T} F={F}", flush=True)
    _hip.qkv_attention_short(xd, packed, rope, mode, batch, T, F, O)
    # the library's unfused pair on the same inputs
    Qd, Kd, Vd, Gd = _hip.seq_buffers(mode, batch, T, F)
    O2 = torch.empty(n, 512, dtype=torch.bfloat16, device=DEV)
    _hip.qkv_rope_gemm(xd, packed, rope, mode, batch, T, F, Qd, Kd, Vd, Gd)
    _hip.attention(Qd, Kd, Vd, Gd, O2, mode, batch, T, F)
    torch.cuda.synchronize()
    assert torch.isfinite(O.float()).all(), "every token's output is written"
    assert_bf16_close(Oref, O, "O fused", min_snr=48)
    s_pair = snr_db(O2.double().cpu().numpy(), O.double().cpu().numpy())
    same = float((O == O2).float().mean())
    print(f"  vs oracle {snr_db(Oref.double().numpy(), O.double().cpu().numpy()):.1f} dB, vs unfused pair "
          f"{s_pair:.1f} dB ({100 * same:.2f}% bitwise equal)")
    assert s_pair >= 55.0


def test_fused_short_attention_rejects_long_sequences(sharp_layers):
    w, packed = sharp_layers[1]
    xn = torch.zeros(65 * 2, 256, dtype=torch.bfloat16, device=DEV)
    O = torch.empty(65 * 2, 512, dtype=torch.bfloat16, device=DEV)
    rope = rope_table(w["freqs"], 65).to(DEV)
    with pytest.raises(ValueError):
        _hip.qkv_attention_short(xn, packed, rope, 1, 1, 2, 65, O)
    lib = _hip.load()
    assert lib.trf_qkv_attention_short(xn.data_ptr(), packed.data_ptr(), rope.data_ptr(), 1, 1, 2, 65,
                                       O.data_ptr(), None) == 1
    assert "at most 64" in lib.trf_last_error().decode()


@pytest.mark.parametrize("F_big,fused", [(16912, True), (16913, False)])
def test_time_sequences_with_a_large_token_stride(sharp_layers, F_big, fused):
    """Time-mode sequences of 63 frames with a token stride of F = 16,912 / 16,913 bands.  The fused kernel
    addresses a sequence's output rows with 32-bit buffer offsets and drops padded positions' stores at
    byte 2^30; at F = 16,913 the sequence's rows ((62 F + 1) KB) would reach past that offset.  There the
    per-op entry point refuses the shape and the block takes the unfused pair; at 16,912 both still take
    the fused kernel.  Bands 0, 8,456 and F - 1 of the block's update are checked against the same bands
    run alone (3 bands, the fused kernel): bitwise where both are fused, >= 55 dB (the fused kernel vs the
    unfused pair) otherwise."""
    w, packed = sharp_layers[0]
    T, n = 63, 63 * F_big
    rope = rope_table(w["freqs"], T).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(77)
    X = torch.randn(n, 256, generator=g, device=DEV)
    sel = torch.tensor([0, 8456, F_big - 1], device=DEV)
    Xs = X.view(T, F_big, 256)[:, sel].reshape(-1, 256).contiguous()
    x_in = Xs.clone()
    print(f"large-stride time block T={T} F={F_big} fused={fused}", flush=True)
    ws = torch.empty(_hip.workspace_bytes(1, T, F_big), dtype=torch.uint8, device=DEV)
    _hip.attn_block(X, 1, T, F_big, packed, 0, rope, ws)
    ws_s = torch.empty(_hip.workspace_bytes(1, T, 3), dtype=torch.uint8, device=DEV)
    _hip.attn_block(Xs, 1, T, 3, packed, 0, rope, ws_s)
    xn = torch.zeros(n, 256, dtype=torch.bfloat16, device=DEV)
    O = torch.empty(n, 512, dtype=torch.bfloat16, device=DEV)
    if fused:
        _hip.qkv_attention_short(xn, packed, rope, 0, 1, T, F_big, O)
    else:
        with pytest.raises(RuntimeError, match="32-bit output offsets"):
            _hip.qkv_attention_short(xn, packed, rope, 0, 1, T, F_big, O)
    torch.cuda.synchronize()
    big = X.view(T, F_big, 256)[:, sel].reshape(-1, 256)
    assert torch.isfinite(big).all()
    upd_big, upd_small = (big - x_in).double().cpu().numpy(), (Xs - x_in).double().cpu().numpy()
    s = snr_db(upd_small, upd_big)
    print(f"  update of bands {sel.tolist()} vs those bands alone: {s:.1f} dB")
    if fused:
        assert torch.equal(big, Xs)
    else:
        assert s >= 55.0
