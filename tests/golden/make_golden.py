"""Write golden vectors of the reference BS-RoFormer (LoggeL/turbo-roformer) for the oracle's tests.

Runs only where the reference sources are present (/root/reference).  It builds the reference module
``turbo_roformer.model.BSRoformer`` with the tiny test configuration, loads this repository's seeded
weights into it with ``strict=True`` (which also pins the state-dict layout), and records:

* ``tiny_forward.npz``: input audio (2 channels, 4000 samples) -> reference forward output, and the
  complex mask the restructured forward feeds to the iSTFT (``FastBSRoformer._mask``);
* ``tiny_stack.npz``: band-split tokens of a 385-sample clip (4 frames x 29 bands) -> output of the
  restructured fp32 stack ``FastBSRoformer._transformer_torch``;
* weight checksums (per-key sum and sum of squares), so a drift of the seeded generator is caught.

Only data is written (inputs and expected outputs); no reference code is copied.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(ROOT / "turbo-roformer_amd"), "/root/reference/src"]

from turbo_roformer.fast import FastBSRoformer  # noqa: E402  (reference)
from turbo_roformer.model import BSRoformer  # noqa: E402  (reference)
from turbo_roformer_amd import signals, weights  # noqa: E402

SEED = 0


def build():
    cfg = weights.TINY_CFG
    m = BSRoformer(cfg["dim"], **{k: v for k, v in cfg.items() if k != "dim"})
    sd = weights.init_state_dict(cfg, seed=SEED)
    m.load_state_dict(sd, strict=True)
    return m.eval(), sd


@torch.inference_mode()
def main() -> None:
    torch.manual_seed(0)
    model, sd = build()
    fast = FastBSRoformer(model, dtype=torch.float32, glue="torch", attn="sdpa", fused=())

    raw = torch.from_numpy(signals.noise_mix(4000, seed=11))[None]
    out = model(raw)
    # the mask fed to the iSTFT by the restructured forward, computed from the same stack output
    st = torch.view_as_real(torch.stft(raw.reshape(2, -1), **model.stft_kwargs, window=model.stft_window_fn(),
                                       return_complex=True))
    nb, T = st.shape[1], st.shape[2]
    xin = st.permute(1, 0, 2, 3).reshape(1, nb * 2, T, 2).permute(0, 2, 1, 3).reshape(1, T, nb * 2 * 2)
    X = model.band_split(xin)
    F = X.shape[2]
    Xs = fast._transformer_torch(X.reshape(T * F, 256).contiguous(), T, F)
    Xn = Xs / Xs.norm(dim=-1, keepdim=True).clamp_min(1e-12) * fast.final_g
    mask = fast._mask(Xn.view(T, F, 256), T, F)
    np.savez(HERE / "tiny_forward.npz", audio=raw.numpy(), output=out.numpy(), mask=mask.numpy(),
             frames=T, bands=F, seed=SEED)

    raw2 = torch.from_numpy(signals.noise_mix(385, seed=12))[None]
    st2 = torch.view_as_real(torch.stft(raw2.reshape(2, -1), **model.stft_kwargs, window=model.stft_window_fn(),
                                        return_complex=True))
    nb2, T2 = st2.shape[1], st2.shape[2]
    xin2 = st2.permute(1, 0, 2, 3).reshape(1, nb2 * 2, T2, 2).permute(0, 2, 1, 3).reshape(1, T2, nb2 * 2 * 2)
    X2 = model.band_split(xin2).reshape(-1, 256).contiguous()
    Y2 = fast._transformer_torch(X2.clone(), T2, X2.shape[0] // T2)
    np.savez(HERE / "tiny_stack.npz", audio=raw2.numpy(), tokens_in=X2.numpy(), tokens_out=Y2.numpy(),
             frames=T2, bands=X2.shape[0] // T2)

    keys = sorted(sd)
    np.savez(HERE / "tiny_weights_checksum.npz", keys=np.array(keys),
             sums=np.array([float(sd[k].double().sum()) for k in keys]),
             sumsq=np.array([float(sd[k].double().pow(2).sum()) for k in keys]),
             n_params=sum(p.numel() for p in model.parameters()))
    print("wrote", [p.name for p in HERE.glob("*.npz")])


if __name__ == "__main__":
    main()
