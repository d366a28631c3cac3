"""Song separation with the stack on the GPU (the Separator's hip backend).

* tiny model, a 4-chunk song: the separated audio against the fp32 forward of the oracle, run through
  the same chunk schedule and overlap-add;
* the full-size model on a 3 s song (one short chunk, 301 frames): audio SNR against the oracle;
* the full-size model at the reference registry's dim_t = 1700 (749,259-sample chunks) on one chunk:
  audio SNR against the oracle;
* the 4:12 synthetic song with the full-size model and 17 s chunks (29 chunks, one batched stack
  forward of 29 x 62 sequences of 1701 frames): identical to the song run in batches of 4 chunks, finite,
  and the schedule of the reference; its first chunk's mask and audio against the fp32 oracle forward of
  that chunk (configuration 5's quality figure); the default batch, sized to the free device memory,
  covers the song;
* three threads sharing one Separator get the single-threaded result bit for bit (the reference's
  tests/test_separator.py:143-157), through ``separate`` and through ``forward_chunks`` on three streams.
"""

from __future__ import annotations

import threading
import time

import numpy as np
import pytest
import torch

from oracle import reference
from turbo_roformer_amd import signals, weights
from turbo_roformer_amd.chunking import overlap_add, step_for
from turbo_roformer_amd.separator import Separator

from .conftest import snr_db

pytestmark = pytest.mark.gpu


def _oracle_song(x: np.ndarray, sd, cfg, chunk: int) -> np.ndarray:
    xt = torch.from_numpy(x)
    return overlap_add(xt, chunk, 2.0, lambda c: reference.forward(c, sd, cfg), batch=1).numpy()


def test_tiny_song_matches_oracle(hip, tiny_sd):
    cfg = weights.TINY_CFG
    sep = Separator(tiny_sd, cfg, weights.TINY_DIM_T, "cuda")
    x = signals.song(40000 / 44100, seed=5)
    print(f"tiny song {x.shape[1]} samples, {sep.n_chunks(x.shape[1])} chunks", flush=True)
    out = sep.separate(x)
    ref = _oracle_song(x, tiny_sd, cfg, sep.chunk)
    assert out.shape == x.shape and out.dtype == np.float32
    s = snr_db(ref, out)
    print(f"  audio snr vs fp32 oracle {s:.1f} dB")
    assert s >= 50.0
    # batching the chunks changes the launch count; the stack itself is batch-invariant bit for bit, but
    # the host GEMMs (band split, mask head) pick other kernels per batch size, and their last-bit fp32
    # differences move a few bf16 roundings in the stack
    out1 = Separator(tiny_sd, cfg, weights.TINY_DIM_T, "cuda", batch_chunks=1).separate(x)
    assert snr_db(out, out1) >= 60.0


@pytest.fixture(scope="module")
def full_sd():
    return weights.init_state_dict(weights.RESURRECTION_CFG, seed=3, init="default", perturb=True)


def test_full_model_short_song_matches_oracle(hip, full_sd):
    cfg = weights.RESURRECTION_CFG
    sep = Separator(full_sd, cfg, 1701, "cuda")
    x = signals.song(3.0, seed=6)
    print(f"full model, 3 s song ({x.shape[1]} samples)", flush=True)
    out = sep.separate(x)
    ref = _oracle_song(x, full_sd, cfg, sep.chunk)
    s = snr_db(ref, out)
    print(f"  audio snr vs fp32 oracle {s:.1f} dB")
    assert s >= 50.0


def test_full_song_batched(hip, full_sd):
    cfg = weights.RESURRECTION_CFG
    x = signals.song(252.0, seed=7)
    sep = Separator(full_sd, cfg, 1701, "cuda", batch_chunks=0)
    assert sep.chunk == 749700 and sep.n_chunks(x.shape[1]) == 29
    print("4:12 song, 29 chunks in one batched stack forward", flush=True)
    sep.separate(x[:, : sep.chunk])  # warm-up (workspace, tables)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = sep.separate(x)
    t1 = time.perf_counter()
    print(f"  {t1 - t0:.2f} s for 252 s of audio (RTF {(t1 - t0) / 252:.4f})")
    assert out.shape == x.shape and np.isfinite(out).all()
    sep4 = Separator(full_sd, cfg, 1701, "cuda", batch_chunks=4)
    out4 = sep4.separate(x)
    assert snr_db(out, out4) >= 60.0
    assert 0.01 < float(np.abs(out).max()) < 10.0


def test_full_song_batched_quality(hip, full_sd):
    """Configuration 5's quality figure (the reference's --quality-seconds, benchmarks/bench_synthetic.py:
    82-84): the 4:12 song separated as one batch of 29 chunks, its first chunk checked against the fp32
    oracle forward of that chunk.  The batch's mask for chunk 0 >= 55 dB against the oracle's mask, the
    batch's prediction for chunk 0 and the song's samples before chunk 1's start (covered by chunk 0
    alone) >= 50 dB against the oracle's audio."""
    cfg = weights.RESURRECTION_CFG
    x = signals.song(252.0, seed=7)
    sep = Separator(full_sd, cfg, 1701, "cuda", batch_chunks=0)
    masks, preds = [], []
    head, fwd = sep.mask_head, sep._forward_chunks

    def mask_head(X, n_frames):
        m = head(X, n_frames)
        masks.append(m.float().cpu())
        return m

    def forward_chunks(chunks):
        y = fwd(chunks)
        preds.append(y.float().cpu())
        return y

    sep.mask_head, sep._forward_chunks = mask_head, forward_chunks
    print("4:12 song, 29 chunks in one batch: chunk 0 against the fp32 oracle", flush=True)
    out = sep.separate(x)
    assert len(preds) == 1 and preds[0].shape[0] == 29, "one batch of 29 chunks"
    T, width = 1701, masks[0].shape[1]
    mask0 = masks[0].view(29, T, width)[0]
    raw = torch.from_numpy(np.ascontiguousarray(x[:, : sep.chunk]))[None]  # chunk 0 starts at sample 0
    Y = reference.stack(reference.stack_input(raw, full_sd, cfg), full_sd, cfg["depth"])
    mask_ref = reference.mask_from_stack(Y, full_sd, cfg)
    audio_ref = reference.apply_mask(raw, mask_ref, cfg)[0].numpy()
    s_mask = snr_db(mask_ref[0].numpy(), mask0.numpy())
    s_pred = snr_db(audio_ref, preds[0][0].numpy())
    half = step_for(sep.chunk, 2.0)  # chunk 1's start
    s_song = snr_db(audio_ref[:, :half], out[:, :half])
    print(f"  chunk 0: mask {s_mask:.1f} dB, prediction {s_pred:.1f} dB, song's first {half} samples "
          f"{s_song:.1f} dB vs fp32 oracle")
    assert s_mask >= 55.0
    assert s_pred >= 50.0 and s_song >= 50.0


def test_full_model_dim_t_1700_matches_oracle(hip, full_sd):
    """The reference's real chunk length: dim_t = 1700, one 749,259-sample chunk (T = 1700, whose last
    time-attention key tile is partly masked)."""
    cfg = weights.RESURRECTION_CFG
    sep = Separator(full_sd, cfg, weights.RESURRECTION_DIM_T, "cuda")
    assert sep.chunk == 749259
    x = signals.song(sep.chunk / 44100, seed=8)
    assert x.shape[1] == sep.chunk and sep.n_chunks(x.shape[1]) == 1
    print("full model, dim_t = 1700, one chunk", flush=True)
    out = sep.separate(x)
    ref = _oracle_song(x, full_sd, cfg, sep.chunk)
    s = snr_db(ref, out)
    print(f"  audio snr vs fp32 oracle {s:.1f} dB")
    assert s >= 50.0


def test_default_batch_fits_device_memory(hip, full_sd):
    cfg = weights.RESURRECTION_CFG
    sep = Separator(full_sd, cfg, 1701, "cuda")
    per = sep.chunk_bytes()
    free, total = torch.cuda.mem_get_info()
    b = sep.batch_size(11_113_200)
    print(f"  {per / 1e9:.2f} GB per chunk, batch of {b} chunks on a {total / 1e9:.0f} GB device")
    assert 0.6e9 < per < 2.0e9
    assert 1 <= b and b * per <= total
    assert Separator(full_sd, cfg, 1701, "cuda", batch_chunks=3).batch_size(11_113_200) == 3


def _threaded(n, fn):
    results = [None] * n
    errors = []

    def work(i):
        try:
            results[i] = fn(i)
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(n)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    return results


def test_concurrent_calls_are_serialised(hip, tiny_sd):
    sep = Separator(tiny_sd, weights.TINY_CFG, weights.TINY_DIM_T, "cuda")
    x = signals.song(40000 / 44100, seed=14)
    expected = sep.separate(x)
    print("3 threads x separate() on one Separator", flush=True)
    for r in _threaded(3, lambda i: sep.separate(x)):
        np.testing.assert_array_equal(r, expected)


def test_concurrent_forward_chunks_on_three_streams(hip, tiny_sd):
    """forward_chunks returns device tensors without waiting: each call waits for the previous one's work
    on the device before it reuses the instance's workspace, whatever stream either ran on."""
    sep = Separator(tiny_sd, weights.TINY_CFG, weights.TINY_DIM_T, "cuda")
    chunks = torch.from_numpy(np.stack([signals.song(sep.chunk / 44100, seed=s) for s in (15, 16)]))
    expected = sep.forward_chunks(chunks).cpu()
    streams = [torch.cuda.Stream() for _ in range(3)]

    def call(i):
        with torch.cuda.stream(streams[i]):
            y = sep.forward_chunks(chunks)
            streams[i].synchronize()
            return y.cpu()

    print("3 threads x forward_chunks() on three streams", flush=True)
    for r in _threaded(3, call):
        assert torch.equal(r, expected)
