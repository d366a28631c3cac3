"""The AVX512-BF16 CPU stack (oracle/cpu_stack.cpp), the same-host CPU baseline, against the fp32 oracle.

It is timed as the kernel-class CPU baseline, so it must compute the same stack:
* full-width sub-layers (256-d tokens, 8 heads of 64, FF 1024) of the full-size model's first two blocks
  on small grids, against ``folded.stack`` (fp32): the SNR of what the stack adds, ``stack(X) - X``,
  >= 44 dB and not below the bf16 torch emulation of the same arithmetic by more than 1 dB.  The
  output itself is mostly the residual X: with the rotary left out of one sub-layer the output still
  reads ~51 dB, the added part ~34 dB, so the bar is on the added part;
* grids with one frame (time sequences of length 1), one band, and lengths past one 64-key tile and
  past a multiple of 16 and of 2 (the padded keys of a tile, the odd key of the last key pair);
* a token's result does not depend on the thread count or on the other chunks of the batch (bitwise);
* argument errors.
Skipped where the CPU has no AVX512-BF16.
"""

from __future__ import annotations

import pytest
import torch

from oracle import cpu_stack, folded
from turbo_roformer_amd import weights

from .conftest import snr_db

pytestmark = pytest.mark.skipif(not cpu_stack.supported(), reason="CPU without AVX512-BF16")

FULL = weights.RESURRECTION_CFG


@pytest.fixture(scope="module")
def layers():
    sd = weights.init_state_dict(FULL, seed=3, init="default", perturb=True)
    return folded.fold(sd, 2)


@pytest.fixture(scope="module")
def stack(layers):
    return cpu_stack.CpuStack(layers, threads=4)


def _x(b, T, F, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(b, T, F, 256, generator=g) * (1 + torch.rand(b, T, F, 1, generator=g) * 4)


@pytest.mark.parametrize("shape", [(1, 37, 5), (1, 1, 3), (1, 17, 1), (1, 65, 63), (2, 19, 6)],
                         ids=["37x5", "one-frame", "one-band", "65x63", "batch2"])
def test_matches_fp32_oracle(stack, layers, shape):
    X = _x(*shape, seed=sum(shape))
    got = stack(X)
    ref = folded.stack(X, layers)
    emu = folded.stack(X, layers, dtype=torch.bfloat16)
    d_ref = (ref - X).numpy()
    s, s_emu = snr_db(d_ref, (got - X).numpy()), snr_db(d_ref, (emu - X).numpy())
    print(f"{shape}: added part {s:.1f} dB (bf16 torch emulation {s_emu:.1f} dB), "
          f"output {snr_db(ref.numpy(), got.numpy()):.1f} dB")
    assert got.shape == X.shape
    assert s >= 44.0
    assert s >= s_emu - 1.0


def test_thread_count_and_batch_independence(stack):
    X = _x(3, 23, 7, seed=11)
    one = stack(X, threads=1)
    assert torch.equal(stack(X, threads=5), one)
    assert torch.equal(stack(X[1:2].contiguous(), threads=2), one[1:2])


def test_phase_seconds_and_errors(stack, layers):
    stack(_x(1, 9, 4, seed=2))
    ph = stack.phase_seconds()
    assert set(ph) == set(cpu_stack.PHASES) and all(v >= 0 for v in ph.values()) and ph["attention"] > 0
    with pytest.raises(ValueError):
        stack(torch.zeros(1, 4, 4, 128))
    assert stack(torch.zeros(1, 0, 4, 256)).shape == (1, 0, 4, 256)
    bad = dict(layers[0], Wo=layers[0]["Wo"][:, :256])
    with pytest.raises(ValueError):
        cpu_stack.CpuStack([bad])
    lib = cpu_stack.load()
    assert lib.trfc_new(0) is None
    assert lib.trfc_forward(None, None, 1, 1, 1, 1) == -1
    h = lib.trfc_new(1)
    try:  # a sub-layer that was never set
        x = torch.zeros(1, 2, 2, 256)
        assert lib.trfc_forward(h, cpu_stack._fp(x), 1, 2, 2, 1) == -2
    finally:
        lib.trfc_free(h)
