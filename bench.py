"""Benchmark of the BS-RoFormer transformer stack on one MI355X.

Workload: one 17 s stereo chunk at 44.1 kHz (749,700 samples, n_fft 2048 / hop 441 -> 1701 frames),
band-split into 62 bands of 256-d tokens, through the 24 sub-layers of the 12-block stack (time attention
+ FF, freq attention + FF) with seeded random weights.  A step is one whole stack forward on the chunk's
tokens, resident in HBM (a device copy restores the input before each step, inside the timed region).

Prints one JSON line: stack forwards/s, the time-attention kernel's TFLOP/s against the bf16 dense MFMA
peak (measured with HIP events on the launch stream over the timed region), and a CPU baseline timed on
the host's cores for one stack forward of the same chunk: the oracle's AVX512-BF16 CPU stack (bf16
operands, fp32 accumulators, the arithmetic of the reference's CPU kernels), with the fp32 restructured
torch path beside it, whose output also gives the mask SNR of the GPU path.

The mask head after the stack (final norm + 62 band MLPs + GLU, one HIP kernel) is timed on the chunk's
stack output beside it, with its own CPU time (the oracle's fp32 mask estimator) and accuracy.

The band split before the stack (62 band RMSNorms + Linears, one HIP kernel) produces the chunk's tokens on
the GPU and is timed the same way.

It also separates a synthetic 4:12 song end to end (for the 29 chunks: one band-split launch, one batched
stack forward and one mask-head launch on the GPU, STFT / iSTFT in PyTorch on the GPU, the Hamming
overlap-add as a HIP kernel) and reports its real-time factor.

    python bench.py [--steps K] [--warmup W] [--precision ff_fp16|ff_split|bf16] [--no-cpu] [--no-song]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "turbo-roformer_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import numpy as np  # noqa: E402
import torch  # noqa: E402

SAMPLES = 749_700  # 17 s at 44.1 kHz -> 1701 frames at hop 441
SONG_SECONDS = 252.0  # the 4:12 song: 29 chunks of 17 s at overlap 2
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


TRAFFIC_SUMMARY = ROOT / "profiles" / "attention_time_17s_chunk_hbm_traffic.md"
KERNEL_STATS = ROOT / "profiles" / "stack_17s_chunk_kernel_stats.md"
COPY_CALIBRATION_BYTES = 1 << 30  # one plain 1 GiB device copy: 1 GiB read + 1 GiB written


def attn_flops(nseq: int, L: int) -> float:
    """Algorithmic FLOPs of one attention call: QK^T and PV, 2*L*L*64 each, per (sequence, head)."""
    return 4.0 * nseq * 8 * L * L * 64


def measured_traffic() -> float | None:
    """HBM bytes per time-attention launch from the committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary
    (each pass already scaled by the same counter's reading for a plain copy of known size), or None."""
    try:
        for line in TRAFFIC_SUMMARY.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch ="):
                return float(line.split("=", 1)[1])
    except OSError:
        pass
    return None


def trace_avg_ms(kernel: str) -> float | None:
    """A kernel's average launch time (ms) in the committed rocprofv3 --kernel-trace --stats summary (its
    table row | `kernel` | calls | avg (us) | ...), or None."""
    try:
        for line in KERNEL_STATS.read_text().splitlines():
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 3 and cells[0] == f"`{kernel}`":
                return float(cells[2]) * 1e-3
    except (OSError, ValueError):
        pass
    return None


def host_cpu() -> dict:
    """The host CPU the baseline runs on: model name, logical CPUs this process may use, physical cores
    (distinct (package, core) pairs in /proc/cpuinfo) and whether it has AVX512-BF16."""
    info = {"model": "unknown", "cpus_usable": len(os.sched_getaffinity(0))}
    try:
        text = Path("/proc/cpuinfo").read_text()
    except OSError:
        return info
    cores, pkg, flags = set(), "0", ""
    for line in text.splitlines():
        key, _, val = line.partition(":")
        key, val = key.strip(), val.strip()
        if key == "model name" and info["model"] == "unknown":
            info["model"] = val
        elif key == "physical id":
            pkg = val
        elif key == "core id":
            cores.add((pkg, val))
        elif key == "flags" and not flags:
            flags = val
    info["physical_cores"] = len(cores) or None
    info["avx512_bf16"] = "avx512_bf16" in flags.split()
    return info


def tune_malloc() -> None:
    """glibc: keep large blocks on the heap (the reference's tune_malloc, separator.py:32-54)."""
    try:
        import ctypes

        libc = ctypes.CDLL("libc.so.6")
        libc.mallopt(-4, 0)  # M_MMAP_MAX
        libc.mallopt(-1, 2_000_000_000)  # M_TRIM_THRESHOLD
    except (OSError, AttributeError):
        pass


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and mask-SNR leg")
    ap.add_argument("--no-song", action="store_true", help="skip the end-to-end 4:12 song separation")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--precision", choices=("ff_fp16", "ff_split", "bf16"), default="ff_fp16",
                    help="FF GEMM arithmetic: fp16 operands (default), split-bf16 operands, or all-bf16 as the "
                         "reference kernels")
    ap.add_argument("--no-alt-precisions", action="store_true",
                    help="time only --precision (the other two stack precisions are skipped)")
    ap.add_argument("--mfma-peak", action="store_true",
                    help="only run the MFMA-rate probe (libtrf_probe.so) and print its JSON line")
    ap.add_argument("--hbm-probe", action="store_true",
                    help="only run the HBM stream-bandwidth probe (libtrf_probe.so) and print its JSON line")
    ap.add_argument("--coissue-probe", action="store_true",
                    help="only run the MFMA/VALU co-issue probe (libtrf_probe.so) and print its JSON line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one plain 1 GiB device copy, the known-size reference for HBM counters")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the stack runs on a single MI355X (no multi-GPU path is built)",
              file=sys.stderr)
        return 2

    if a.mfma_peak or a.hbm_probe or a.coissue_probe:
        # the instruction-throughput and bandwidth figures the roofline fractions are read against (the
        # reference's counterpart: benchmarks/dpbf16_peak.cpp)
        from turbo_roformer_amd import probe

        out = {"probe": "MI355X sustained rates", "device": torch.cuda.get_device_name(0)}
        if a.mfma_peak:
            out["mfma_bf16_32x32x16"] = probe.mfma_peak()
        if a.hbm_probe:
            out["hbm_stream"] = probe.hbm_stream()
        if a.coissue_probe:
            out["mfma_valu_coissue"] = probe.coissue()
        print(json.dumps(out), flush=True)
        return 0

    from turbo_roformer_amd import _hip, signals, weights
    from turbo_roformer_amd.band_split import HipBandSplit
    from turbo_roformer_amd.host import HostPath
    from turbo_roformer_amd.stack import HipStack

    cfg = weights.RESURRECTION_CFG
    sd = weights.init_state_dict(cfg, seed=a.seed, init="default", perturb=True)
    host = HostPath(sd, cfg, "cpu")
    raw = torch.from_numpy(signals.noise_mix(SAMPLES, seed=a.seed))[None]
    feats = host.spectrogram(raw)  # (1, T, bins * 2 * 2) fp32
    t_bs = time.perf_counter()
    X0 = host.band_split(feats)  # (1, T, F, 256) fp32, torch on the host
    band_cpu_s = time.perf_counter() - t_bs
    _, T, F, _ = X0.shape
    # the step before the stack on the GPU: band split of the chunk's features into the stack's tokens
    bsplit = HipBandSplit(sd, cfg, "cuda")
    fd = feats.reshape(T, -1).contiguous().cuda()
    Xd0 = bsplit(fd)
    for _ in range(3):
        bsplit(fd, out=Xd0)
    torch.cuda.synchronize()
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b0.record()
    for _ in range(20):
        bsplit(fd, out=Xd0)
    b1.record()
    torch.cuda.synchronize()
    band_ms = b0.elapsed_time(b1) / 20
    band_snr = signals.snr_db(X0.reshape(-1, 256).numpy(), Xd0.cpu().numpy())
    del fd

    if a.copy_calibration:
        src = torch.ones(COPY_CALIBRATION_BYTES // 4, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def slot_names(mode: int) -> dict[int, str]:
        """Kernel of each slot of a sub-layer: sequences of at most 64 positions (frequency attention at
        62 bands) run QKV and attention as one fused kernel, reported in the attention slot."""
        L = T if mode == 0 else F
        if L <= 64:
            return {1: "qkv_attention_short", 2: "post_attention"}
        return {0: "qkv_rope_gemm", 1: "attention", 2: "post_attention"}

    def make_events(stack, steps: int, want) -> list:
        """Per step, the trf_stack_forward_timed event list: an Event pair for each (layer, slot) that
        want(mode, slot) selects, None elsewhere (the library records nothing for None)."""
        nslot = len(_hip.SLOTS)
        out = []
        for _ in range(steps):
            evs = [None] * (2 * nslot * len(stack.layers))
            for i, mode in enumerate(stack.modes):
                for sl in slot_names(mode):
                    if want(mode, sl):
                        evs[2 * (i * nslot + sl)] = torch.cuda.Event(enable_timing=True)
                        evs[2 * (i * nslot + sl) + 1] = torch.cuda.Event(enable_timing=True)
            for e in evs:  # create the underlying events outside the timed region
                if e is not None:
                    e.record()
            out.append(evs)
        torch.cuda.synchronize()
        return out

    def per_kernel_ms(stack, events) -> dict[str, float]:
        nslot = len(_hip.SLOTS)
        acc: dict[str, list[float]] = {}
        for evs in events:
            for i, mode in enumerate(stack.modes):
                for sl, name in slot_names(mode).items():
                    e0, e1 = evs[2 * (i * nslot + sl)], evs[2 * (i * nslot + sl) + 1]
                    if e0 is not None:
                        acc.setdefault(f"{name}_{'t' if mode == 0 else 'f'}", []).append(e0.elapsed_time(e1))
        return {k: float(np.mean(v)) for k, v in acc.items()}

    def timed(precision: str, with_events: bool):
        """(ms per stack forward, per-kernel ms or None, time-attention ms or None, output) for one
        precision.  In the timed forwards only the time-attention kernels (the roofline kernel) carry
        events, attached to their dispatch; the per-kernel table comes from as many forwards after them,
        with events on every kernel (each event pair adds a few microseconds between kernels)."""
        stack = HipStack(sd, "cuda", precision=precision)
        X = torch.empty_like(Xd0)
        for _ in range(a.warmup):
            X.copy_(Xd0)
            stack(X, 1, T, F)
        torch.cuda.synchronize()
        timed_events = make_events(stack, a.steps, lambda mode, sl: with_events and mode == 0 and sl == 1)
        t0 = time.perf_counter()
        for k in range(a.steps):
            X.copy_(Xd0)
            stack(X, 1, T, F, events=timed_events[k] if with_events else None)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms = (t1 - t0) * 1e3 / a.steps
        print(f"bench: {a.steps} timed stack forwards ({precision}), {ms:.3f} ms each", file=sys.stderr, flush=True)
        kernel_ms = attn_ms = None
        out = X.view(1, T, F, 256).cpu()
        if with_events:
            attn_ms = per_kernel_ms(stack, timed_events)["attention_t"]
            prof_events = make_events(stack, a.steps, lambda mode, sl: True)
            for k in range(a.steps):
                X.copy_(Xd0)
                stack(X, 1, T, F, events=prof_events[k])
            torch.cuda.synchronize()
            kernel_ms = per_kernel_ms(stack, prof_events)
        del stack, X
        torch.cuda.empty_cache()
        return ms, kernel_ms, attn_ms, out

    ms, kernel_ms, attn_t_ms, out_gpu = timed(a.precision, True)
    alts = {p: timed(p, False) for p in ("ff_fp16", "ff_split", "bf16")
            if p != a.precision and not a.no_alt_precisions}

    # the mask head after the stack, on this chunk's stack output (HIP events on its launch stream)
    from turbo_roformer_amd.mask import HipMaskHead

    head = HipMaskHead(sd, cfg, "cuda")
    mask_of = lambda x: head(x.reshape(-1, 256).contiguous().cuda(), x.shape[1]).cpu().view(1, x.shape[1], -1)
    xg = out_gpu.reshape(-1, 256).cuda()
    mask_buf = torch.empty(T, head.width, device="cuda")
    for _ in range(3):
        head(xg, T, mask_buf)
    torch.cuda.synchronize()
    m0, m1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 20
    m0.record()
    for _ in range(reps):
        head(xg, T, mask_buf)
    m1.record()
    torch.cuda.synchronize()
    mask_ms = m0.elapsed_time(m1) / reps
    mask_flops = 2 * T * (F * 256 * head.hidden + head.hidden * 2 * head.width)
    result_mask = {"kernel": "mask head (final norm + 62 band MLPs + GLU), split-fp16 MFMA", "ms_per_chunk": round(mask_ms, 4),
                   "gflop_per_chunk": round(mask_flops / 1e9, 2),
                   "tflops": round(mask_flops / (mask_ms * 1e-3) / 1e12, 1)}
    del xg, mask_buf
    flops_t = attn_flops(F, T)
    achieved = flops_t / (attn_t_ms * 1e-3) / 1e12
    # the same figure from the committed kernel trace's average (profiles/), for a reader to recompute
    trace_ms = trace_avg_ms("trf::k_attn_long")

    result = {
        "metric": "17s-chunk stack forwards/sec; time-attn TFLOP/s and % of bf16 MFMA peak",
        "value": round(1e3 / ms, 3),
        "unit": "stack forwards/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16+fp16",
        "dtype_detail": ("bf16 MFMA operands for the QKV GEMM, both attentions and the out-projection; fp16 "
                         "operands for the two feed-forward GEMMs (ff_fp16); fp32 accumulation, residual stream, "
                         "norms, rotary and softmax statistics") if a.precision == "ff_fp16" else a.precision,
        "data": "synthetic (seeded Gaussian + pink-noise stereo mix, peak 0.5; seeded random weights)",
        "config": {
            "workload": "BS-RoFormer 12-block transformer stack (24 sub-layers) on one 17 s chunk",
            "samples": SAMPLES, "frames": T, "bands": F, "tokens": T * F, "dim": 256, "heads": 8, "head_dim": 64,
            "ff_hidden": 1024, "chunks": 1,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "attention (time, 62 x 8 sequences of 1701 frames)",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(),
            "flops_per_launch": flops_t,
            "avg_launch_ms": round(attn_t_ms, 4),
            "trace_avg_launch_ms": None if trace_ms is None else round(trace_ms, 4),
            "frac_trace": None if trace_ms is None else round(flops_t / (trace_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "frac_trace_source": str(KERNEL_STATS.relative_to(ROOT)),
        },
        "kernels_ms_per_launch": {k: round(v, 4) for k, v in sorted(kernel_ms.items())},
        "precision": a.precision,
        "other_precisions": {p: {"ms_per_step": round(v[0], 4), "value": round(1e3 / v[0], 3)} for p, v in alts.items()},
        "mask_head": result_mask,
        "band_split": {"kernel": "band split (62 band RMSNorm + Linear, fp32 MFMA)", "ms_per_chunk": round(band_ms, 4),
                       "torch_cpu_ms_per_chunk": round(band_cpu_s * 1e3, 1),
                       "snr_db_vs_torch_fp32": round(band_snr, 2)},
    }

    if not a.no_song:
        # whole synthetic 4:12 song: 29 chunks of 17 s at overlap 2; band split, one batched stack forward and
        # the mask head on the kernels, STFT and iSTFT in PyTorch on the same GPU, Hamming overlap-add on the CPU
        from turbo_roformer_amd.separator import Separator

        sep = Separator(sd, cfg, T, "cuda", stack_precision=a.precision, batch_chunks=0)
        song = signals.song(SONG_SECONDS, seed=a.seed)
        sep.separate(song[:, : sep.chunk])  # warm-up: tables, workspace
        torch.cuda.synchronize()
        t4 = time.perf_counter()
        sep.separate(song)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t4
        print(f"bench: {SONG_SECONDS:.0f} s song separated in {wall:.3f} s", file=sys.stderr, flush=True)
        result["song"] = {"audio_s": SONG_SECONDS, "chunks": sep.n_chunks(song.shape[1]), "wall_s": round(wall, 3),
                          "rtf": round(wall / SONG_SECONDS, 5), "overlap": 2.0}
        if not a.no_cpu:
            # quality on the song's first chunk (the reference's --quality-seconds, bench_synthetic.py:78-84):
            # the same separation by the fp32 oracle forward, same chunk schedule and overlap-add
            from oracle import reference
            from turbo_roformer_amd.chunking import overlap_add

            head_n = sep.chunk
            print(f"bench: song quality, fp32 oracle on the first {head_n / 44100:.1f} s", file=sys.stderr,
                  flush=True)
            fast = sep.separate(song[:, :head_n])
            exact = overlap_add(torch.from_numpy(np.ascontiguousarray(song[:, :head_n])), sep.chunk, 2.0,
                                lambda c: reference.forward(c, sd, cfg), batch=1).numpy()
            result["song"]["quality_seconds"] = round(head_n / 44100, 2)
            result["song"]["snr_vs_fp32_db"] = round(signals.snr_db(exact, fast), 2)
        del sep

    if not a.no_cpu:
        from oracle import cpu_stack, folded, reference

        tune_malloc()
        threads = torch.get_num_threads()
        cpu_info = host_cpu()
        layers = folded.fold(sd, cfg["depth"])
        print(f"bench: cpu baseline, one fp32 stack forward on {threads} threads", file=sys.stderr, flush=True)
        t2 = time.perf_counter()
        ref = folded.stack(X0, layers)
        t3 = time.perf_counter()
        cpu_s = t3 - t2
        snr_x = signals.snr_db(ref.numpy(), out_gpu.numpy())
        t5 = time.perf_counter()
        m_ref = reference.mask_from_stack(ref, sd, cfg)
        mask_cpu_s = time.perf_counter() - t5
        # the product path: HIP stack, then the HIP mask head
        m_gpu = mask_of(out_gpu)
        snr_mask = signals.snr_db(m_ref.numpy(), m_gpu.numpy())
        snr_alts = {p: signals.snr_db(m_ref.numpy(), mask_of(v[3]).numpy()) for p, v in alts.items()}
        result["mask_head"]["cpu_ms_per_chunk"] = round(mask_cpu_s * 1e3, 1)
        result["mask_head"]["cpu_sample"] = f"oracle fp32 mask estimator on {threads} threads, one chunk"
        # the head alone: HIP mask head on the fp32 stack output against the fp32 mask estimator
        result["mask_head"]["head_snr_db_vs_fp32"] = round(signals.snr_db(m_ref.numpy(), mask_of(ref).numpy()), 2)
        # the reference's published ratio of its fp32 restructured torch stack to its AVX512-BF16 kernel
        # stack, both stack only: attention + feed-forward blocks 17.89 + 6.46 s against the default
        # kernel path's stack sections 6.07 s per chunk (docs/benchmarks.md:104-112)
        kernel_ratio = (17.89 + 6.46) / 6.07
        torch_fp32 = {"s_per_forward": round(cpu_s, 2), "gpu_speedup": round((1e3 / ms) * cpu_s, 1),
                      "reference_kernel_ratio": round(kernel_ratio, 2),
                      "reference_kernel_ratio_scope": "stack only (docs/benchmarks.md:104-112)",
                      "kernel_equivalent_s": round(cpu_s / kernel_ratio, 2),
                      "gpu_speedup_vs_kernel_equivalent": round((1e3 / ms) * cpu_s / kernel_ratio, 1)}
        print(f"bench: cpu baseline, one bf16 (oneDNN GEMMs + SDPA) stack forward on {threads} threads",
              file=sys.stderr, flush=True)
        t7 = time.perf_counter()
        y_b16 = folded.stack_bf16_sdpa(X0, layers)
        b16_s = time.perf_counter() - t7
        torch_bf16 = {"s_per_forward": round(b16_s, 2), "gpu_speedup": round((1e3 / ms) * b16_s, 1),
                      "mask_snr_db_vs_fp32": round(signals.snr_db(
                          m_ref.numpy(), reference.mask_from_stack(y_b16, sd, cfg).numpy()), 2)}
        del y_b16
        if cpu_stack.supported():
            # the kernel-class CPU baseline: the AVX512-BF16 stack (bf16 operands, fp32 accumulators), one
            # warm-up forward (it grows and first-touches its work buffers), then the best of three
            cs = cpu_stack.CpuStack(layers, threads)
            print(f"bench: cpu baseline, AVX512-BF16 stack forwards on {threads} threads", file=sys.stderr,
                  flush=True)
            cs(X0)
            ph0 = cs.phase_seconds()
            runs = []
            for _ in range(3):
                t6 = time.perf_counter()
                y_cpu = cs(X0)
                runs.append(time.perf_counter() - t6)
            ph1 = cs.phase_seconds()
            cpu_k_s = min(runs)
            m_cpu = reference.mask_from_stack(y_cpu, sd, cfg)
            result["cpu_baseline"] = {
                "value": round(1.0 / cpu_k_s, 5),
                "unit": "stack forwards/s",
                "cores": threads,
                "kind": "port",
                "sample": f"one stack forward (24 sub-layers, {T}x{F} tokens) of the AVX512-BF16 CPU stack "
                          f"(oracle/cpu_stack.cpp: vdpbf16ps GEMMs and attention with fused epilogues, bf16 "
                          f"operands, fp32 accumulators and residual), best of {len(runs)} after a warm-up, "
                          f"{cpu_k_s:.2f} s",
                "gpu_speedup": round((1e3 / ms) * cpu_k_s, 1),
                "mask_snr_db_vs_fp32": round(signals.snr_db(m_ref.numpy(), m_cpu.numpy()), 2),
                "phase_s": {k: round((ph1[k] - ph0[k]) / len(runs), 3) for k in cpu_stack.PHASES},
                "host": cpu_info,
                "torch_fp32": torch_fp32,
                "torch_bf16": torch_bf16,
            }
        else:
            result["cpu_baseline"] = {
                "value": round(1.0 / cpu_s, 5),
                "unit": "stack forwards/s",
                "cores": threads,
                "kind": "port",
                "sample": f"one fp32 stack forward (24 sub-layers, {T}x{F} tokens) of the restructured torch "
                          f"path (fast.py _transformer_torch restated), {cpu_s:.1f} s; this CPU has no "
                          f"AVX512-BF16 for the kernel-class CPU stack",
                "gpu_speedup": torch_fp32["gpu_speedup"],
                "host": cpu_info,
                "torch_fp32": torch_fp32,
                "torch_bf16": torch_bf16,
            }
        result["parity"] = {"mask_snr_db_vs_fp32": round(snr_mask, 2), "stack_out_snr_db_vs_fp32": round(snr_x, 2)}
        for p, v in snr_alts.items():
            result["parity"][f"mask_snr_db_vs_fp32_{p}"] = round(v, 2)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
