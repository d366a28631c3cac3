"""Per-op parity of the gfx950 kernels (through the C ABI) against the oracle's kernel emulations.

Shapes cover both attention regimes (short L <= 64 single-pass, long L > 64 two-pass), odd and ragged
lengths (one key past a 64-key tile, L = 1, the 1700/1701-frame chunk), batching, and the padded
positions the kernels must zero.  Tolerance: within two bf16 steps elementwise (one rounding-boundary
flip allowed in 1e-4 of the elements) and a per-op SNR floor.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import folded, kernels as ok
from turbo_roformer_amd import _hip, weights
from turbo_roformer_amd.stack import rope_table

from .conftest import assert_bf16_close, rand_x, snr_db

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def layers(hip):
    """Two folded sub-layers (time, freq) of a seeded model with N(0,0.02) weights and perturbed gains."""
    cfg = dict(weights.TINY_CFG, depth=1)
    sd = weights.init_state_dict(cfg, seed=3, init="normal")
    out = []
    for P in folded.fold(sd, 1):
        w = ok.bf16_weights(P)
        packed = torch.empty(_hip.layer_packed_bytes(), dtype=torch.uint8, device=DEV)
        dev = dict(
            w_qkvg=w["W"].to(DEV), b_gate=w["b_gate"].to(DEV), w_out=w["Wo"].to(DEV), w_ff1=w["W1"].to(DEV),
            b_ff1=w["b1"].to(DEV), w_ff2=w["W2"].to(DEV), b_ff2=w["b2"].to(DEV),
        )
        _hip.pack_layer(**dev, out=packed)
        out.append((w, packed))
    torch.cuda.synchronize()
    return out


def _xn(n, seed):
    return ok.l2_rows(rand_x(n, seed)).to(torch.bfloat16)


@pytest.mark.parametrize("y", [None, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_add_rmsnorm(hip, y, out_dtype):
    n = 1003
    X = rand_x(n, 1, 3.0)
    Y = None if y is None else rand_x(n, 2).to(y)
    ref_x, ref_out = ok.add_rmsnorm(X, Y, out_dtype)
    Xd = X.to(DEV)
    out = torch.empty(n, 256, dtype=out_dtype, device=DEV)
    print(f"add_rmsnorm n={n} y={y} out={out_dtype}", flush=True)
    _hip.add_rmsnorm(Xd, None if Y is None else Y.to(DEV), out)
    torch.cuda.synchronize()
    torch.testing.assert_close(Xd.cpu(), ref_x, rtol=1e-6, atol=1e-6)
    if out_dtype == torch.bfloat16:
        assert_bf16_close(ref_out, out, "add_rmsnorm", min_snr=60)
    else:
        torch.testing.assert_close(out.cpu(), ref_out, rtol=1e-5, atol=1e-7)


QKV_SHAPES = [  # (mode, batch, T, F)
    (0, 1, 100, 7),
    (1, 1, 100, 7),
    (1, 2, 37, 62),
    (0, 1, 65, 3),
    (0, 1, 64, 3),
    (0, 2, 1, 5),
    (1, 1, 5, 1),
    (0, 1, 1701, 2),
    (1, 1, 9, 62),
]


# (0, 1, 1701, 40): 270 blocks of 256 rows, 3,510 (block, stage) units, so each of the kernel's
# workgroups (one per CU) runs 13-14 stages back to back across block boundaries.
@pytest.mark.parametrize("mode,batch,T,F", QKV_SHAPES + [(0, 1, 1701, 40)])
def test_qkv_rope_gemm(hip, layers, mode, batch, T, F):
    w, packed = layers[mode]
    n = batch * T * F
    xn = _xn(n, 10 + T)
    L = T if mode == 0 else F
    rope = rope_table(w["freqs"], L)
    Qr, Kr, Vr, Gr = ok.qkv_rope(xn, w["W"], w["b_gate"], w["freqs"], mode, batch, T, F)
    Q, K, Vt, G = _hip.seq_buffers(mode, batch, T, F)
    for t in (Q, K, Vt):
        t.fill_(1.0)  # pads must be overwritten with zeros
    print(f"qkv_rope_gemm mode={mode} batch={batch} T={T} F={F}", flush=True)
    _hip.qkv_rope_gemm(xn.to(DEV), packed, rope.to(DEV), mode, batch, T, F, Q, K, Vt, G)
    torch.cuda.synchronize()
    assert_bf16_close(Qr, Q, "Q")
    assert_bf16_close(Kr, K, "K")
    assert_bf16_close(Vr, Vt, "Vt")
    torch.testing.assert_close(G.cpu(), Gr, rtol=2e-5, atol=2e-6)
    assert (Q.cpu()[:, :, :, L:] == 0).all() and (K.cpu()[:, :, :, L:] == 0).all() and (Vt.cpu()[..., L:] == 0).all()


# (0, 1, 300, 100): 1,600 workgroups of time attention (three rounds on 256 CUs at two per CU); the second
# query block of each sequence has one wave with queries and three without.
ATT_SHAPES = QKV_SHAPES + [(0, 1, 1700, 2), (0, 1, 200, 9), (1, 3, 11, 64), (0, 1, 300, 100)]


@pytest.mark.parametrize("mode,batch,T,F", ATT_SHAPES)
def test_attention(hip, layers, mode, batch, T, F):
    w, _ = layers[mode]
    n = batch * T * F
    # sharper attention than unit-norm inputs give: scale xn so scores span tens of units
    xn = (ok.l2_rows(rand_x(n, 20 + T)) * 1.0).to(torch.bfloat16)
    Wq = w["W"].float().clone()
    Wq[:1024] *= 6.0
    Q, K, Vt, G = ok.qkv_rope(xn, Wq.to(torch.bfloat16), w["b_gate"], w["freqs"], mode, batch, T, F)
    Oref = ok.attention(Q, K, Vt, G, mode, batch, T, F)
    O = torch.empty(n, 512, dtype=torch.bfloat16, device=DEV)
    print(f"attention mode={mode} batch={batch} T={T} F={F}", flush=True)
    _hip.attention(Q.to(DEV), K.to(DEV), Vt.to(DEV), G.to(DEV), O, mode, batch, T, F)
    torch.cuda.synchronize()
    assert_bf16_close(Oref, O, "O", min_snr=48)
    # against textbook fp64 softmax attention on the same bf16 operands (no bf16 P): SNR only.
    # Q carries log2(e), so the natural-log scores are q.k * ln 2.
    L = T if mode == 0 else F
    idx = ok.token_index(mode, batch, T, F)
    q, k = ok.qk_rows(Q)[:, :, :L].double(), ok.qk_rows(K)[:, :, :L].double()
    v = Vt[:, :, :, :L].double().transpose(-1, -2)
    o = torch.softmax((q @ k.transpose(-1, -2)) * math.log(2.0), dim=-1) @ v
    o = o * G[idx].permute(0, 2, 1).unsqueeze(-1).double()
    exact = torch.empty(n, 8, 64, dtype=torch.float64)
    exact[idx] = o.permute(0, 2, 1, 3)
    assert snr_db(exact.view(n, 512).numpy(), O.double().cpu().numpy()) >= 40.0


@pytest.mark.parametrize("T,F,key,spiked", [(900, 2, 700, (96, 128)), (400, 64, 300, (96, 128)),
                                            (900, 2, 700, (96, 112)), (900, 2, 700, (112, 128))])
def test_attention_far_above_the_first_keys_takes_the_guarded_sweep(hip, layers, T, F, key, spiked):
    """Long sequences are swept with a fixed integer shift from the first 32 keys; a score far above it
    overflows that sweep's sums, and the sweep is redone with the raised-shift method.  Here the queries
    `spiked` of every (sequence, head) are a multiple of one key, so their scores on it are ~100 (base 2)
    above the rest: the result must still be the softmax.  With F = 64, 512 of the 1,024 workgroups redo
    their sweep.  96..127 is one 32-query column tile; the half tiles 96..111 and 112..127 raise the
    shift of queries j and j + 16 of a tile differently, whose row sums one lane holds together."""
    w, _ = layers[0]
    mode, batch = 0, 1
    n = batch * T * F
    xn = ok.l2_rows(rand_x(n, 77)).to(torch.bfloat16)
    Q, K, Vt, G = ok.qkv_rope(xn, w["W"], w["b_gate"], w["freqs"], mode, batch, T, F)
    K[:, :, :, key, :] = 4.0
    Q[:, :, :, spiked[0]:spiked[1], :] = 100.0 / (64 * 16.0) * 4.0  # q . k_key = 64 * 4 * 0.39 = 100
    Oref = ok.attention(Q, K, Vt, G, mode, batch, T, F)
    O = torch.empty(n, 512, dtype=torch.bfloat16, device=DEV)
    print("attention with a dominant key (guarded sweep)", flush=True)
    _hip.attention(Q.to(DEV), K.to(DEV), Vt.to(DEV), G.to(DEV), O, mode, batch, T, F)
    torch.cuda.synchronize()
    assert torch.isfinite(O.float()).all()
    assert_bf16_close(Oref, O, "O", min_snr=48)
    # the spiked queries attend to the one key alone: O = gate * V[key]
    idx = ok.token_index(mode, batch, T, F)  # [nseq, L] token of (sequence, position)
    for s_ in range(idx.shape[0]):
        tok = idx[s_, spiked[0] + 4]
        vk = Vt[s_, :, :, key].float()  # [8 heads, 64]
        want = (G[tok].float()[:, None] * vk).reshape(512)
        torch.testing.assert_close(O[tok].float().cpu(), want, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("which", ["out", "ff2", "k256"])
@pytest.mark.parametrize("n", [1, 31, 1000, 4133])
def test_gemm_res_norm(hip, layers, which, n):
    """gemm_res_norm(A, Wp, bias?, X, xn, eps) with a standalone packed weight: the out-projection (K = 512,
    no bias), FF2 (K = 1024, bias) and a K = 256 weight of its own, as the reference op takes any K."""
    w, _ = layers[0]
    if which == "k256":
        g = torch.Generator().manual_seed(7)
        W, b = (torch.randn(256, 256, generator=g) * 0.05).to(torch.bfloat16), torch.randn(256, generator=g)
    else:
        W, b = (w["Wo"], None) if which == "out" else (w["W2"], w["b2"])
    kd = W.shape[1]
    A = (rand_x(n, 30 + n).repeat(1, kd // 256) * 0.5).to(torch.bfloat16)
    X = rand_x(n, 40 + n, 2.0)
    Xr, xnr = ok.gemm_res_norm(A, W, b, X)
    Xd = X.to(DEV)
    xn = torch.empty(n, 256, dtype=torch.bfloat16, device=DEV)
    print(f"gemm_res_norm {which} K={kd} n={n}", flush=True)
    Wp = _hip.pack_weight(W.to(DEV))
    _hip.gemm_res_norm(A.to(DEV), Wp, None if b is None else b.to(DEV), Xd, xn)
    torch.cuda.synchronize()
    torch.testing.assert_close(Xd.cpu(), Xr, rtol=1e-5, atol=1e-5)
    assert_bf16_close(xnr, xn, "xn", min_snr=55)


@pytest.mark.parametrize("n_out", [1024, 96])
@pytest.mark.parametrize("n", [1, 77, 4096])
def test_gemm_gelu(hip, layers, n, n_out):
    """gemm_gelu(xn, Wp, bias, H) with a standalone packed weight: FF1 (1024 outputs) and the first 96 rows
    of it (the op takes any multiple of 32 outputs)."""
    w, _ = layers[1]
    W1, b1 = w["W1"][:n_out].contiguous(), w["b1"][:n_out].contiguous()
    xn = _xn(n, 50 + n)
    Hr = ok.gemm_gelu(xn, W1, b1)
    H = torch.empty(n, n_out, dtype=torch.bfloat16, device=DEV)
    print(f"gemm_gelu n={n} n_out={n_out}", flush=True)
    _hip.gemm_gelu(xn.to(DEV), _hip.pack_weight(W1.to(DEV)), b1.to(DEV), H)
    torch.cuda.synchronize()
    assert_bf16_close(Hr, H, "H", min_snr=50)


def test_errors_are_raised(hip, layers):
    """Bad arguments come back as RuntimeError with the library's message (no launch)."""
    w, packed = layers[0]
    Q, K, Vt, G = _hip.seq_buffers(0, 1, 8, 2)
    O = torch.empty(16, 512, dtype=torch.bfloat16, device=DEV)
    lib = _hip.load()
    rc = lib.trf_attention(Q.data_ptr(), K.data_ptr(), Vt.data_ptr(), G.data_ptr(), O.data_ptr(), 7, 1, 8, 2, None)
    assert rc == 1 and b"mode" in lib.trf_last_error()
    rc = lib.trf_attention(Q.data_ptr() + 2, K.data_ptr(), Vt.data_ptr(), G.data_ptr(), O.data_ptr(), 0, 1, 8, 2, None)
    assert rc == 1 and b"aligned" in lib.trf_last_error()
    with pytest.raises(ValueError):
        _hip.attention(Q, K, Vt, G, O[:8], 0, 1, 8, 2)
