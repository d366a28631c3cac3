"""trf_stack_forward_static, the stack forward whose workspace is the library's static device array (for
callers that cannot allocate), against trf_stack_forward with a caller-owned workspace: bitwise equal on two
calls in a row, the second on a smaller chunk, and shapes beyond the static array rejected with an error."""

from __future__ import annotations

import pytest
import torch

from turbo_roformer_amd import _hip, weights
from turbo_roformer_amd.stack import HipStack

pytestmark = pytest.mark.gpu
DEV = "cuda"
F = 62


@pytest.fixture(scope="module")
def full_stack(hip):
    sd = weights.init_state_dict(weights.RESURRECTION_CFG, seed=4, init="default", perturb=True)
    return HipStack(sd, DEV)


def _tokens(T: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(T * F, 256, generator=g)


def test_static_workspace_forward_equals_workspace_forward(full_stack):
    s = full_stack
    for T, seed in ((1701, 1), (300, 2)):  # the full 17 s chunk, then a smaller one into the same array
        X = _tokens(T, seed)
        Xa = X.to(DEV)
        Xb = X.to(DEV)
        print(f"static-workspace stack forward T={T}", flush=True)
        s(Xa, 1, T, F)
        _hip.stack_forward_static(Xb, 1, T, F, s.layers, s.modes, s.table(0, T), s.table(1, F), s.precision)
        torch.cuda.synchronize()
        assert torch.isfinite(Xb).all()
        assert torch.equal(Xa, Xb)


def test_static_workspace_rejects_shapes_beyond_it(full_stack):
    s = full_stack
    T = 1701
    assert _hip.workspace_bytes(2, T, F) > _hip.STATIC_WORKSPACE_BYTES
    X = torch.zeros(2 * T * F, 256, device=DEV)
    with pytest.raises(RuntimeError, match="static workspace"):
        _hip.stack_forward_static(X, 2, T, F, s.layers, s.modes, s.table(0, T), s.table(1, F), s.precision)
    assert bool((X == 0).all())  # rejected before any launch


def test_static_workspace_forward_under_graph_capture(full_stack):
    """The allocation-free entry point captured in a HIP graph (torch.cuda.CUDAGraph).  Its first call on a
    device looks the static array's device address up, which has to happen outside a capture, so one eager
    call comes first; the captured forward is then replayed three times, X restored and the stream
    synchronised between replays, each bitwise equal to the eager forward."""
    s = full_stack
    T = 300
    rt, rf = s.table(0, T), s.table(1, F)
    X0 = _tokens(T, 3).to(DEV)
    Xe = X0.clone()
    print(f"static-workspace stack forward T={T}: eager, then captured and replayed", flush=True)
    _hip.stack_forward_static(Xe, 1, T, F, s.layers, s.modes, rt, rf, s.precision)
    torch.cuda.synchronize()
    Xg = X0.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _hip.stack_forward_static(Xg, 1, T, F, s.layers, s.modes, rt, rf, s.precision)
    torch.cuda.synchronize()
    for r in range(3):
        Xg.copy_(X0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"  replay {r}", flush=True)
        assert torch.equal(Xg, Xe)
