"""The 24-sub-layer BS-RoFormer stack on one MI355X: weight folding, rotary tables, workspace, launch.

``HipStack`` plays the role of the C++ glue of ``FastBSRoformer`` (src/turbo_roformer/fast.py:97-215,
269-341): it folds each sub-layer's norm gains and the attention scale into the following weights
(``_prep``, fast.py:163-191), uploads them, lets the library pack them into MFMA operand order, builds
the fp32 rotary tables on the host exactly as ``_tables`` does (fast.py:193-201) and runs the stack
through ``trf_stack_forward``.  Work buffers are allocated once per shape and reused, so one forward
runs at a time per instance (the reference's instances have the same rule, fast.py:24).

Precision (the feed-forward GEMMs only; attention, QKV and the out-projection are bf16 in every mode):
``"bf16"`` rounds every GEMM operand to bf16, the arithmetic of the reference kernels (~48 dB mask SNR
against the fp32 forward on seeded random weights).  ``"ff_fp16"`` (the default) gives the two FF GEMMs
fp16 operands at the same speed (~58 dB).  ``"ff_split"`` gives them split-bf16 operands, three
products each (~59 dB, slower).
"""

from __future__ import annotations

from collections.abc import Mapping

import torch

from . import _hip

H, DH, DIM = _hip.HEADS, _hip.HEAD_DIM, _hip.DIM


def fold_sublayer(sd: Mapping[str, torch.Tensor], prefix: str) -> dict[str, torch.Tensor]:
    """Plain folded weights of one (attention, feed-forward) pair, fp32 on the host.

    ``prefix`` is e.g. ``"layers.3.1.layers.0"``.  Folding (fast.py:163-182): the RMSNorm gain
    ``gamma * sqrt(256)`` of the attention norm multiplies the input columns of W_qkv and W_gate, the
    attention scale 1/8 (exact in bf16) multiplies W_q, and the FF norm gain multiplies W1's columns.
    """
    scale = DIM**0.5
    ga = (sd[f"{prefix}.0.norm.gamma"].float() * scale)[None, :]
    wqkv = sd[f"{prefix}.0.to_qkv.weight"].float() * ga
    wqkv[: H * DH] *= DH**-0.5
    wg = sd[f"{prefix}.0.to_gates.weight"].float() * ga
    gf = (sd[f"{prefix}.1.net.0.gamma"].float() * scale)[None, :]
    return dict(
        w_qkvg=torch.cat([wqkv, wg], 0),
        b_gate=sd[f"{prefix}.0.to_gates.bias"].float(),
        w_out=sd[f"{prefix}.0.to_out.0.weight"].float(),
        w_ff1=sd[f"{prefix}.1.net.1.weight"].float() * gf,
        b_ff1=sd[f"{prefix}.1.net.1.bias"].float(),
        w_ff2=sd[f"{prefix}.1.net.4.weight"].float(),
        b_ff2=sd[f"{prefix}.1.net.4.bias"].float(),
    )


def sublayer_prefixes(sd: Mapping[str, torch.Tensor]) -> list[tuple[str, int]]:
    """(prefix, mode) of every sub-layer in execution order: block i time (mode 0), then freq (mode 1)."""
    out = []
    i = 0
    while f"layers.{i}.0.layers.0.0.to_qkv.weight" in sd:
        for mode in (0, 1):
            if f"layers.{i}.{mode}.layers.1.0.to_qkv.weight" in sd:
                raise NotImplementedError("only time/freq transformer depth 1 is supported")
            out.append((f"layers.{i}.{mode}.layers.0", mode))
        i += 1
    if not out:
        raise ValueError("state dict has no transformer layers")
    return out


def rope_table(freqs: torch.Tensor, L: int) -> torch.Tensor:
    """[2, L, 32] fp32 (cos, sin) of angle p * freq_i, computed in fp32 on the host (fast.py:193-201)."""
    pos = torch.arange(L, dtype=torch.float32)
    ang = pos[:, None] * freqs.detach().float().cpu()[None, :]
    return torch.stack((ang.cos(), ang.sin())).contiguous()


class HipStack:
    """Folded, packed weights of the whole stack on one device, plus cached tables and workspace."""

    def __init__(self, state_dict: Mapping[str, torch.Tensor], device: str | torch.device = "cuda",
                 precision: str = "ff_fp16"):
        _hip.load()
        _hip.precision_code(precision)
        self.precision = precision
        self.device = torch.device(device)
        sd = {k: v.detach() for k, v in state_dict.items()}
        prefixes = sublayer_prefixes(sd)
        self.modes = [m for _, m in prefixes]
        nb = _hip.layer_packed_bytes()
        self.packed = torch.empty(len(prefixes), nb, dtype=torch.uint8, device=self.device)
        for i, (prefix, _) in enumerate(prefixes):
            w = fold_sublayer(sd, prefix)
            for k in ("w_ff1", "w_ff2"):  # bf16 residuals of the fp32 FF weights (split lo parts; fp16 = hi + lo)
                w[k + "_lo"] = w[k] - w[k].to(torch.bfloat16).float()
            dev = {
                k: (v.to(torch.bfloat16) if k.startswith("w_") else v).to(self.device).contiguous()
                for k, v in w.items()
            }
            _hip.pack_layer(
                dev["w_qkvg"], dev["b_gate"], dev["w_out"], dev["w_ff1"], dev["b_ff1"], dev["w_ff2"], dev["b_ff2"],
                self.packed[i], dev["w_ff1_lo"], dev["w_ff2_lo"],
            )
        self.layers = [self.packed[i] for i in range(len(prefixes))]
        self.freqs = {
            0: sd["layers.0.0.layers.0.0.rotary_embed.freqs"].float().clone(),
            1: sd["layers.0.1.layers.0.0.rotary_embed.freqs"].float().clone(),
        }
        self._tables: dict[tuple[int, int], torch.Tensor] = {}
        self._ws: torch.Tensor | None = None
        torch.cuda.synchronize(self.device)

    @classmethod
    def from_model(cls, model: torch.nn.Module, device="cuda", precision: str = "ff_fp16") -> HipStack:
        """From a loaded reference ``BSRoformer`` module (or anything with the same state-dict keys)."""
        return cls(model.state_dict(), device, precision)

    def table(self, mode: int, L: int) -> torch.Tensor:
        key = (mode, L)
        if key not in self._tables:
            self._tables[key] = rope_table(self.freqs[mode], L).to(self.device)
        return self._tables[key]

    def workspace(self, batch: int, T: int, F: int) -> torch.Tensor:
        need = _hip.workspace_bytes(batch, T, F)
        if self._ws is None or self._ws.numel() < need:
            self._ws = None
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def release_buffers(self) -> None:
        """Free the cached workspace (re-created on the next call)."""
        self._ws = None

    def forward(self, X: torch.Tensor, batch: int, T: int, F: int, events: list | None = None,
                check_finite: bool = False) -> torch.Tensor:
        """Run all sub-layers on X [batch*T*F, 256] fp32 (token order (c, t, f)) in place and return it.

        X must be finite: a NaN or inf token gives non-finite outputs for its sequences (every kernel still
        runs its fixed number of steps, so nothing hangs).  ``check_finite=True`` checks X on the device
        first and raises ValueError (this waits for the device, so it is off by default; ``Separator``
        rejects non-finite audio before the STFT instead).
        ``events``: optional per-kernel timing events (see ``_hip.stack_forward``)."""
        if check_finite and not bool(torch.isfinite(X).all()):
            raise ValueError("X contains NaN or inf")
        _hip.stack_forward(
            X, batch, T, F, self.layers, self.modes, self.table(0, T), self.table(1, F), self.workspace(batch, T, F),
            events, self.precision,
        )
        return X

    __call__ = forward

    def attn_block(self, X: torch.Tensor, batch: int, T: int, F: int, layer: int) -> torch.Tensor:
        mode = self.modes[layer]
        L = T if mode == 0 else F
        _hip.attn_block(X, batch, T, F, self.layers[layer], mode, self.table(mode, L), self.workspace(batch, T, F))
        return X

    def ff_block(self, X: torch.Tensor, batch: int, T: int, F: int, layer: int) -> torch.Tensor:
        _hip.ff_block(X, batch, T, F, self.layers[layer], self.workspace(batch, T, F), self.precision)
        return X
