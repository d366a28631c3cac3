"""Loader and thin torch wrappers of the gfx950 C-ABI library ``libtrf_hip.so``.

Counterpart of the reference's kernel loader (src/turbo_roformer/_kernels.py): ``support()`` says
whether the backend can run here, ``load()`` returns the library or raises ``HipUnavailable``
(the analogue of ``KernelUnavailable``, _kernels.py:27-28), and the op wrappers below mirror the
reference's ``torch.ops.turbo_roformer.*`` ops (kernels.cpp:644-652) on device tensors.

The library is built in-tree (``make -C turbo-roformer_amd/csrc``); it shares PyTorch's HIP runtime
(same soname), so every call is enqueued on ``torch.cuda.current_stream()``.
"""

from __future__ import annotations

import ctypes
import os
import re
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).with_name("libtrf_hip.so")
HEADER_PATH = Path(__file__).resolve().parents[2] / "include" / "trf_hip.h"
ABI_VERSION = 8
STATIC_WORKSPACE_BYTES = 512 << 20  # TRF_STATIC_WORKSPACE_BYTES of trf_hip.h

DIM, HEADS, HEAD_DIM, QKVG_ROWS, FF_HIDDEN = 256, 8, 64, 1544, 1024
MODE_TIME, MODE_FREQ = 0, 1
PREC_BF16, PREC_FF_SPLIT, PREC_FF_FP16 = 0, 1, 2
PRECISIONS = {"bf16": PREC_BF16, "ff_split": PREC_FF_SPLIT, "ff_fp16": PREC_FF_FP16}
MASK_SPLIT, MASK_FP16 = 0, 1
MASK_PRECISIONS = {"split": MASK_SPLIT, "fp16": MASK_FP16}
_F32, _BF16 = 0, 1

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class HipUnavailable(RuntimeError):
    """The gfx950 HIP backend cannot be used here (reason in the message)."""


class TrfLayerSrc(ctypes.Structure):
    """``trf_layer_src`` of trf_hip.h: device pointers to one sub-layer's plain folded weights."""

    _fields_ = [
        ("w_qkvg", ctypes.c_void_p),
        ("b_gate", ctypes.c_void_p),
        ("w_out", ctypes.c_void_p),
        ("w_ff1", ctypes.c_void_p),
        ("b_ff1", ctypes.c_void_p),
        ("w_ff2", ctypes.c_void_p),
        ("b_ff2", ctypes.c_void_p),
        ("w_ff1_lo", ctypes.c_void_p),
        ("w_ff2_lo", ctypes.c_void_p),
    ]


class TrfMaskBandSrc(ctypes.Structure):
    """``trf_mask_band_src`` of trf_hip.h: device pointers to one band's mask-estimator MLP weights."""

    _fields_ = [("w1", ctypes.c_void_p), ("b1", ctypes.c_void_p), ("w2", ctypes.c_void_p), ("b2", ctypes.c_void_p)]


class TrfBandSplitSrc(ctypes.Structure):
    """``trf_band_split_src`` of trf_hip.h: device pointers to one band's RMSNorm gain and Linear."""

    _fields_ = [("w", ctypes.c_void_p), ("b", ctypes.c_void_p), ("gamma", ctypes.c_void_p)]


_P, _I32, _I64, _F, _SZ = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
_SIGNATURES: dict[str, tuple] = {
    "trf_abi_version": (ctypes.c_int, []),
    "trf_last_error": (ctypes.c_char_p, []),
    "trf_seq_pad": (_I32, [_I32]),
    "trf_seq_buffer_elems": (_I64, [_I32, _I32, _I32, _I32]),
    "trf_layer_packed_bytes": (_SZ, []),
    "trf_pack_layer": (ctypes.c_int, [ctypes.POINTER(TrfLayerSrc), _P, _P]),
    "trf_add_rmsnorm": (ctypes.c_int, [_P, _P, _I32, _P, _I32, _I64, _F, _P]),
    "trf_qkv_rope_gemm": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P]),
    "trf_attention": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _P]),
    "trf_qkv_attention_short": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _P, _P]),
    "trf_weight_packed_bytes": (_SZ, [_I32, _I32]),
    "trf_pack_weight": (ctypes.c_int, [_P, _I32, _I32, _P, _P]),
    "trf_gemm_res_norm": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _I64, _F, _P]),
    "trf_gemm_gelu": (ctypes.c_int, [_P, _P, _P, _I32, _P, _I64, _P]),
    "trf_stack_workspace_bytes": (_SZ, [_I32, _I32, _I32]),
    "trf_stack_forward": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int32), _I32, _I32, _P, _P, _P,
         _SZ, _P],
    ),
    "trf_stack_forward_timed": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int32), _I32, _I32, _P, _P, _P,
         _SZ, ctypes.POINTER(ctypes.c_void_p), _I32, _P],
    ),
    "trf_stack_forward_static": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int32), _I32, _I32, _P, _P, _P],
    ),
    "trf_attn_block": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _I32, _P, _P, _SZ, _P]),
    "trf_ff_block": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _I32, _P, _SZ, _P]),
    "trf_band_split_packed_bytes": (_SZ, [ctypes.POINTER(ctypes.c_int32), _I32]),
    "trf_pack_band_split": (
        ctypes.c_int, [ctypes.POINTER(TrfBandSplitSrc), ctypes.POINTER(ctypes.c_int32), _I32, _P, _P]
    ),
    "trf_band_split": (ctypes.c_int, [_P, _I32, _I32, ctypes.POINTER(ctypes.c_int32), _P, _P, _P]),
    "trf_overlap_add": (ctypes.c_int, [_P, _I32, _I64, _I32, _P, _P, _I64, _P, _P, _P]),
    "trf_overlap_finish": (ctypes.c_int, [_P, _P, _I64, _F, _P, _P]),
    "trf_mask_head_packed_bytes": (_SZ, [ctypes.POINTER(ctypes.c_int32), _I32, _I32]),
    "trf_pack_mask_head": (
        ctypes.c_int, [ctypes.POINTER(TrfMaskBandSrc), ctypes.POINTER(ctypes.c_int32), _I32, _I32, _P, _P, _P]
    ),
    "trf_mask_head": (ctypes.c_int, [_P, _I32, _I32, ctypes.POINTER(ctypes.c_int32), _I32, _P, _I32, _P, _P]),
}


def header_functions(path: Path = HEADER_PATH) -> list[str]:
    """Names of the functions declared in trf_hip.h."""
    text = re.sub(r"/\*.*?\*/", " ", path.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(trf_[a-z_0-9]+)\s*\(", text)))


def open_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    """dlopen the library and declare argument types; needs no GPU (used by the symbol checks)."""
    if not path.exists():
        raise HipUnavailable(f"{path.name} is not built (run `make -C turbo-roformer_amd/csrc`)")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.trf_abi_version() != ABI_VERSION:
        raise HipUnavailable(f"ABI version {lib.trf_abi_version()} != {ABI_VERSION}")
    return lib


def support() -> tuple[bool, str]:
    """(usable, reason): library present, a ROCm GPU visible, and that GPU is a gfx950."""
    if os.environ.get("TURBO_ROFORMER_DISABLE_HIP"):
        return False, "disabled by TURBO_ROFORMER_DISABLE_HIP"
    if not LIB_PATH.exists():
        return False, f"{LIB_PATH.name} is not built"
    if torch.version.hip is None:
        return False, "this PyTorch has no ROCm support"
    if not torch.cuda.is_available():
        return False, "no ROCm GPU is visible"
    arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
    if not arch.startswith("gfx950"):
        return False, f"device is {arch}, the kernels are built for gfx950"
    return True, f"gfx950 ({torch.cuda.get_device_name()})"


def load() -> ctypes.CDLL:
    """The library, ready to launch on the current device.  Raises HipUnavailable."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        ok, reason = support()
        if not ok:
            raise HipUnavailable(reason)
        torch.cuda.init()  # the library must bind to torch's HIP runtime, loaded first
        _lib = open_library()
        return _lib


def is_loaded() -> bool:
    return _lib is not None


def _check(rc: int) -> None:
    if rc != 0:
        msg = _lib.trf_last_error().decode() if _lib is not None else "unknown error"
        raise RuntimeError(f"trf error {rc}: {msg}")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple | None = None) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


# ---------------------------------------------------------------------------------------------- shapes


def seq_pad(L: int) -> int:
    return (L + 63) // 64 * 64


def seq_shape(mode: int, batch: int, T: int, F: int) -> tuple[int, int, int]:
    """(number of sequences, length, padded length) of an attention mode."""
    nseq, L = (batch * F, T) if mode == MODE_TIME else (batch * T, F)
    return nseq, L, seq_pad(L)


def layer_packed_bytes() -> int:
    return int(load().trf_layer_packed_bytes())


def workspace_bytes(batch: int, T: int, F: int) -> int:
    n = load().trf_stack_workspace_bytes(batch, T, F)
    if n == 0:
        _check(1)
    return int(n)


# ---------------------------------------------------------------------------------------------- ops


def precision_code(precision: str) -> int:
    if precision not in PRECISIONS:
        raise ValueError(f"precision must be one of {tuple(PRECISIONS)}, got {precision!r}")
    return PRECISIONS[precision]


def pack_layer(w_qkvg, b_gate, w_out, w_ff1, b_ff1, w_ff2, b_ff2, out: torch.Tensor, w_ff1_lo=None,
               w_ff2_lo=None) -> None:
    """Pack plain folded weights (device, row-major) into ``out`` (uint8, layer_packed_bytes()).

    ``w_ff1_lo`` / ``w_ff2_lo``: optional bf16 residuals ``w - bf16(w)`` of the fp32 FF weights, for the
    ``ff_split`` precision (zero when omitted)."""
    lib = load()
    _need(w_qkvg, "w_qkvg", torch.bfloat16, (QKVG_ROWS, DIM))
    _need(b_gate, "b_gate", torch.float32, (HEADS,))
    _need(w_out, "w_out", torch.bfloat16, (DIM, HEADS * HEAD_DIM))
    _need(w_ff1, "w_ff1", torch.bfloat16, (FF_HIDDEN, DIM))
    _need(b_ff1, "b_ff1", torch.float32, (FF_HIDDEN,))
    _need(w_ff2, "w_ff2", torch.bfloat16, (DIM, FF_HIDDEN))
    _need(b_ff2, "b_ff2", torch.float32, (DIM,))
    _need(out, "out", torch.uint8, (lib.trf_layer_packed_bytes(),))
    if w_ff1_lo is not None:
        _need(w_ff1_lo, "w_ff1_lo", torch.bfloat16, (FF_HIDDEN, DIM))
    if w_ff2_lo is not None:
        _need(w_ff2_lo, "w_ff2_lo", torch.bfloat16, (DIM, FF_HIDDEN))
    src = TrfLayerSrc(*(t.data_ptr() for t in (w_qkvg, b_gate, w_out, w_ff1, b_ff1, w_ff2, b_ff2)),
                      _ptr(w_ff1_lo), _ptr(w_ff2_lo))
    _check(lib.trf_pack_layer(ctypes.byref(src), out.data_ptr(), _stream()))


def add_rmsnorm(X: torch.Tensor, Y: torch.Tensor | None, out: torch.Tensor, eps: float = 1e-12) -> None:
    """X += Y (optional); out = X / max(|X|, eps) per row (kernels.cpp:101-137)."""
    lib = load()
    _need(X, "X", torch.float32)
    if X.dim() != 2 or X.shape[1] != DIM:
        raise ValueError(f"X must be [n, {DIM}]")
    ydt = _F32
    if Y is not None:
        _need(Y, "Y", Y.dtype, tuple(X.shape))
        if Y.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("Y must be float32 or bfloat16")
        ydt = _BF16 if Y.dtype == torch.bfloat16 else _F32
    _need(out, "out", out.dtype, tuple(X.shape))
    if out.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out must be float32 or bfloat16")
    odt = _BF16 if out.dtype == torch.bfloat16 else _F32
    _check(lib.trf_add_rmsnorm(X.data_ptr(), _ptr(Y), ydt, out.data_ptr(), odt, X.shape[0], eps, _stream()))


def qk_shape(nseq: int, Lp: int) -> tuple[int, ...]:
    """Chunk-major Q/K: [nseq, 8 heads, 8 chunks of 8 features, Lpad, 8] (trf_hip.h)."""
    return (nseq, HEADS, HEAD_DIM // 8, Lp, 8)


def seq_buffers(mode: int, batch: int, T: int, F: int, device="cuda") -> tuple[torch.Tensor, ...]:
    """Q, K [nseq, 8, 8, Lpad, 8] (chunk-major) and Vt [nseq, 8, 64, Lpad] bf16, plus G [ntok, 8] fp32."""
    nseq, L, Lp = seq_shape(mode, batch, T, F)
    Q = torch.empty(qk_shape(nseq, Lp), dtype=torch.bfloat16, device=device)
    K = torch.empty_like(Q)
    Vt = torch.empty(nseq, HEADS, HEAD_DIM, Lp, dtype=torch.bfloat16, device=device)
    G = torch.empty(batch * T * F, HEADS, dtype=torch.float32, device=device)
    return Q, K, Vt, G


def qkv_rope_gemm(xn, layer, rope, mode, batch, T, F, Q, K, Vt, G) -> None:
    """xn [ntok, 256] bf16 -> rotated Q, K, transposed V and sigmoid gates (kernels.cpp:439-540)."""
    lib = load()
    nseq, L, Lp = seq_shape(mode, batch, T, F)
    n = batch * T * F
    _need(xn, "xn", torch.bfloat16, (n, DIM))
    _need(layer, "layer", torch.uint8, (lib.trf_layer_packed_bytes(),))
    _need(rope, "rope", torch.float32, (2, L, HEAD_DIM // 2))
    _need(Q, "Q", torch.bfloat16, qk_shape(nseq, Lp))
    _need(K, "K", torch.bfloat16, qk_shape(nseq, Lp))
    _need(Vt, "Vt", torch.bfloat16, (nseq, HEADS, HEAD_DIM, Lp))
    _need(G, "G", torch.float32, (n, HEADS))
    _check(
        lib.trf_qkv_rope_gemm(
            xn.data_ptr(), layer.data_ptr(), rope.data_ptr(), mode, batch, T, F,
            Q.data_ptr(), K.data_ptr(), Vt.data_ptr(), G.data_ptr(), _stream(),
        )
    )


def attention(Q, K, Vt, G, O, mode, batch, T, F) -> None:
    """Exact softmax attention + gate + head merge into O [ntok, 512] bf16 (kernels.cpp:250-388)."""
    lib = load()
    nseq, L, Lp = seq_shape(mode, batch, T, F)
    n = batch * T * F
    _need(Q, "Q", torch.bfloat16, qk_shape(nseq, Lp))
    _need(K, "K", torch.bfloat16, qk_shape(nseq, Lp))
    _need(Vt, "Vt", torch.bfloat16, (nseq, HEADS, HEAD_DIM, Lp))
    _need(G, "G", torch.float32, (n, HEADS))
    _need(O, "O", torch.bfloat16, (n, HEADS * HEAD_DIM))
    _check(lib.trf_attention(Q.data_ptr(), K.data_ptr(), Vt.data_ptr(), G.data_ptr(), O.data_ptr(), mode, batch, T, F, _stream()))


def qkv_attention_short(xn, layer, rope, mode, batch, T, F, O) -> None:
    """``qkv_rope_gemm`` + ``attention`` fused for sequences of at most 64 positions: xn [ntok, 256] bf16
    -> O [ntok, 512] bf16, no sequence buffers."""
    lib = load()
    nseq, L, Lp = seq_shape(mode, batch, T, F)
    if L > 64:
        raise ValueError(f"sequences of {L} positions: the fused kernel takes at most 64")
    n = batch * T * F
    _need(xn, "xn", torch.bfloat16, (n, DIM))
    _need(layer, "layer", torch.uint8, (lib.trf_layer_packed_bytes(),))
    _need(rope, "rope", torch.float32, (2, L, HEAD_DIM // 2))
    _need(O, "O", torch.bfloat16, (n, HEADS * HEAD_DIM))
    _check(lib.trf_qkv_attention_short(xn.data_ptr(), layer.data_ptr(), rope.data_ptr(), mode, batch, T, F,
                                       O.data_ptr(), _stream()))


def weight_packed_bytes(rows: int, K: int) -> int:
    """Bytes of a weight [rows][K] packed by ``pack_weight``."""
    return int(load().trf_weight_packed_bytes(rows, K))


def pack_weight(W: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Pack a bf16 weight W [rows][K] (device) into the operand tiles the per-op GEMMs read: the
    counterpart of ``_pack_w`` (fast.py:43-49) for ``gemm_res_norm`` / ``gemm_gelu``."""
    lib = load()
    if W.dim() != 2:
        raise ValueError(f"W must be 2-D, got {tuple(W.shape)}")
    rows, K = W.shape
    nbytes = lib.trf_weight_packed_bytes(rows, K)
    if nbytes == 0:
        raise ValueError(f"W [{rows}][{K}]: K must be a positive multiple of 16")
    _need(W, "W", torch.bfloat16, (rows, K))
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=W.device)
    _need(out, "out", torch.uint8, (nbytes,))
    _check(lib.trf_pack_weight(W.data_ptr(), rows, K, out.data_ptr(), _stream()))
    return out


def gemm_res_norm(A, Wp, bias, X, xn, eps: float = 1e-12) -> None:
    """``gemm_res_norm(A, Wp, bias?, X, xn, eps)`` (kernels.cpp:542-586): X += A @ W^T (+ bias) and
    xn = X / max(|X|, eps) as bf16, with W [256][K] packed by ``pack_weight``."""
    lib = load()
    n, K = A.shape
    _need(A, "A", torch.bfloat16, (n, K))
    _need(Wp, "Wp", torch.uint8, (lib.trf_weight_packed_bytes(DIM, K),))
    if bias is not None:
        _need(bias, "bias", torch.float32, (DIM,))
    _need(X, "X", torch.float32, (n, DIM))
    _need(xn, "xn", torch.bfloat16, (n, DIM))
    _check(lib.trf_gemm_res_norm(A.data_ptr(), K, Wp.data_ptr(), _ptr(bias), X.data_ptr(), xn.data_ptr(), n, eps,
                                 _stream()))


def gemm_gelu(xn, Wp, bias, H) -> None:
    """``gemm_gelu(xn, Wp, bias, H)`` (kernels.cpp:609-642): H = gelu_erf(xn @ W^T + bias) as bf16, with
    W [n_out][256] packed by ``pack_weight``."""
    lib = load()
    n, n_out = H.shape
    _need(xn, "xn", torch.bfloat16, (n, DIM))
    _need(Wp, "Wp", torch.uint8, (lib.trf_weight_packed_bytes(n_out, DIM),))
    _need(bias, "bias", torch.float32, (n_out,))
    _need(H, "H", torch.bfloat16, (n, n_out))
    _check(lib.trf_gemm_gelu(xn.data_ptr(), Wp.data_ptr(), bias.data_ptr(), n_out, H.data_ptr(), n, _stream()))


SLOTS = ("qkv_rope_gemm", "attention", "post_attention")  # trf_kernel_slot order


def stack_forward(X, batch, T, F, layers: list[torch.Tensor], modes: list[int], rope_time, rope_freq, ws,
                  events: list | None = None, precision: str = "ff_fp16") -> None:
    """The whole stack on X [batch*T*F, 256] fp32, in place (fast.py:269-341).

    ``precision``: ``"bf16"`` (every GEMM operand bf16, the reference kernels' arithmetic),
    ``"ff_fp16"`` (fp16 operands in the two FF GEMMs) or ``"ff_split"`` (split-bf16 operands there).

    ``events``: optional list of 2*len(SLOTS)*len(layers) ``torch.cuda.Event`` (or None) recorded before/after
    each kernel (slot order ``SLOTS``), for per-kernel timing on the launch stream."""
    lib = load()
    prec = precision_code(precision)
    _need(X, "X", torch.float32, (batch * T * F, DIM))
    _need(ws, "workspace", torch.uint8)
    nb = lib.trf_layer_packed_bytes()
    for i, t in enumerate(layers):
        _need(t, f"layers[{i}]", torch.uint8, (nb,))
    if len(modes) != len(layers):
        raise ValueError("modes and layers differ in length")
    if any(m == MODE_TIME for m in modes):
        _need(rope_time, "rope_time", torch.float32, (2, T, HEAD_DIM // 2))
    if any(m == MODE_FREQ for m in modes):
        _need(rope_freq, "rope_freq", torch.float32, (2, F, HEAD_DIM // 2))
    ptrs = (ctypes.c_void_p * max(1, len(layers)))(*[t.data_ptr() for t in layers])
    mds = (ctypes.c_int32 * max(1, len(modes)))(*modes)
    if events is None:
        _check(
            lib.trf_stack_forward(
                X.data_ptr(), batch, T, F, ptrs, mds, len(layers), prec, _ptr(rope_time), _ptr(rope_freq),
                ws.data_ptr(), ws.numel(), _stream(),
            )
        )
        return
    if len(events) != 2 * len(SLOTS) * len(layers):
        raise ValueError(f"need {2 * len(SLOTS) * len(layers)} events, got {len(events)}")
    handles = []
    for e in events:
        if e is not None and not e.cuda_event:
            e.record()  # materialise the underlying hipEvent_t
        handles.append(None if e is None else e.cuda_event)
    evs = (ctypes.c_void_p * len(handles))(*handles)
    _check(
        lib.trf_stack_forward_timed(
            X.data_ptr(), batch, T, F, ptrs, mds, len(layers), prec, _ptr(rope_time), _ptr(rope_freq),
            ws.data_ptr(), ws.numel(), evs, len(handles), _stream(),
        )
    )


def stack_forward_static(X, batch, T, F, layers: list[torch.Tensor], modes: list[int], rope_time, rope_freq,
                         precision: str = "ff_fp16") -> None:
    """``stack_forward`` with the library's static device workspace (``trf_stack_forward_static``): no
    workspace argument and no device allocation, for callers that cannot allocate.  Calls on one GPU
    share that workspace, so they must not overlap; shapes whose workspace exceeds
    ``STATIC_WORKSPACE_BYTES`` raise."""
    lib = load()
    prec = precision_code(precision)
    _need(X, "X", torch.float32, (batch * T * F, DIM))
    nb = lib.trf_layer_packed_bytes()
    for i, t in enumerate(layers):
        _need(t, f"layers[{i}]", torch.uint8, (nb,))
    if len(modes) != len(layers):
        raise ValueError("modes and layers differ in length")
    if any(m == MODE_TIME for m in modes):
        _need(rope_time, "rope_time", torch.float32, (2, T, HEAD_DIM // 2))
    if any(m == MODE_FREQ for m in modes):
        _need(rope_freq, "rope_freq", torch.float32, (2, F, HEAD_DIM // 2))
    ptrs = (ctypes.c_void_p * max(1, len(layers)))(*[t.data_ptr() for t in layers])
    mds = (ctypes.c_int32 * max(1, len(modes)))(*modes)
    _check(
        lib.trf_stack_forward_static(
            X.data_ptr(), batch, T, F, ptrs, mds, len(layers), prec, _ptr(rope_time), _ptr(rope_freq), _stream(),
        )
    )


def attn_block(X, batch, T, F, layer, mode, rope, ws) -> None:
    """One attention sub-layer X += attn(X) on the residual stream (model.py:141)."""
    lib = load()
    _need(X, "X", torch.float32, (batch * T * F, DIM))
    _need(layer, "layer", torch.uint8, (lib.trf_layer_packed_bytes(),))
    L = T if mode == MODE_TIME else F
    _need(rope, "rope", torch.float32, (2, L, HEAD_DIM // 2))
    _need(ws, "workspace", torch.uint8)
    _check(lib.trf_attn_block(X.data_ptr(), batch, T, F, layer.data_ptr(), mode, rope.data_ptr(), ws.data_ptr(), ws.numel(), _stream()))


def ff_block(X, batch, T, F, layer, ws, precision: str = "ff_fp16") -> None:
    """One feed-forward sub-layer X += ff(X) (model.py:142)."""
    lib = load()
    prec = precision_code(precision)
    _need(X, "X", torch.float32, (batch * T * F, DIM))
    _need(layer, "layer", torch.uint8, (lib.trf_layer_packed_bytes(),))
    _need(ws, "workspace", torch.uint8)
    _check(lib.trf_ff_block(X.data_ptr(), batch, T, F, layer.data_ptr(), prec, ws.data_ptr(), ws.numel(), _stream()))


# ---------------------------------------------------------------------------------------------- mask head


def _dins(dins) -> ctypes.Array:
    return (ctypes.c_int32 * len(dins))(*[int(d) for d in dins])


def mask_head_packed_bytes(dins, hidden: int) -> int:
    """Bytes of the packed mask head for band widths ``dins`` and MLP hidden size ``hidden``."""
    lib = load()
    n = lib.trf_mask_head_packed_bytes(_dins(dins), len(dins), hidden)
    if n == 0:
        _check(1)
    return int(n)


def pack_mask_head(bands: list[tuple[torch.Tensor, ...]], dins, hidden: int, final_gamma: torch.Tensor,
                   out: torch.Tensor) -> None:
    """Pack per-band ``(w1 [hidden, 256], b1 [hidden], w2 [2 din, hidden], b2 [2 din])`` fp32 device
    tensors and the final norm's gamma into ``out`` (uint8, mask_head_packed_bytes())."""
    lib = load()
    if len(bands) != len(dins):
        raise ValueError("bands and dins differ in length")
    for i, ((w1, b1, w2, b2), d) in enumerate(zip(bands, dins)):
        _need(w1, f"w1[{i}]", torch.float32, (hidden, DIM))
        _need(b1, f"b1[{i}]", torch.float32, (hidden,))
        _need(w2, f"w2[{i}]", torch.float32, (2 * d, hidden))
        _need(b2, f"b2[{i}]", torch.float32, (2 * d,))
    _need(final_gamma, "final_gamma", torch.float32, (DIM,))
    _need(out, "out", torch.uint8, (lib.trf_mask_head_packed_bytes(_dins(dins), len(dins), hidden),))
    src = (TrfMaskBandSrc * len(bands))(*[TrfMaskBandSrc(*(t.data_ptr() for t in b)) for b in bands])
    _check(lib.trf_pack_mask_head(src, _dins(dins), len(dins), hidden, final_gamma.data_ptr(), out.data_ptr(),
                                  _stream()))


def mask_head(X: torch.Tensor, n_frames: int, dins, hidden: int, packed: torch.Tensor, mask: torch.Tensor,
              precision: str = "split") -> None:
    """mask [n_frames, sum(dins)] from the stack output X [n_frames * len(dins), 256] fp32: final norm,
    per-band Linear / tanh / Linear / GLU (fast.py:349-360)."""
    lib = load()
    if precision not in MASK_PRECISIONS:
        raise ValueError(f"precision must be one of {tuple(MASK_PRECISIONS)}, got {precision!r}")
    F = len(dins)
    _need(X, "X", torch.float32, (n_frames * F, DIM))
    _need(packed, "packed", torch.uint8, (lib.trf_mask_head_packed_bytes(_dins(dins), F, hidden),))
    _need(mask, "mask", torch.float32, (n_frames, int(sum(dins))))
    _check(lib.trf_mask_head(X.data_ptr(), n_frames, F, _dins(dins), hidden, packed.data_ptr(),
                             MASK_PRECISIONS[precision], mask.data_ptr(), _stream()))


# ---------------------------------------------------------------------------------------------- band split


def band_split_packed_bytes(dins) -> int:
    """Bytes of the packed band split for band widths ``dins``."""
    lib = load()
    n = lib.trf_band_split_packed_bytes(_dins(dins), len(dins))
    if n == 0:
        _check(1)
    return int(n)


def pack_band_split(bands: list[tuple[torch.Tensor, ...]], dins, out: torch.Tensor) -> None:
    """Pack per-band ``(w [256, din], b [256], gamma [din])`` fp32 device tensors into ``out`` (uint8,
    band_split_packed_bytes())."""
    lib = load()
    if len(bands) != len(dins):
        raise ValueError("bands and dins differ in length")
    for i, ((w, b, g), d) in enumerate(zip(bands, dins)):
        _need(w, f"w[{i}]", torch.float32, (DIM, d))
        _need(b, f"b[{i}]", torch.float32, (DIM,))
        _need(g, f"gamma[{i}]", torch.float32, (d,))
    _need(out, "out", torch.uint8, (lib.trf_band_split_packed_bytes(_dins(dins), len(dins)),))
    src = (TrfBandSplitSrc * len(bands))(*[TrfBandSplitSrc(*(t.data_ptr() for t in b)) for b in bands])
    _check(lib.trf_pack_band_split(src, _dins(dins), len(dins), out.data_ptr(), _stream()))


def band_split(feats: torch.Tensor, n_frames: int, dins, packed: torch.Tensor, X: torch.Tensor) -> None:
    """X [n_frames * len(dins), 256] = per-band RMSNorm + Linear of feats [n_frames, sum(dins)] fp32
    (model.py:147-155), in the stack's token order."""
    lib = load()
    F = len(dins)
    _need(feats, "feats", torch.float32, (n_frames, int(sum(dins))))
    _need(packed, "packed", torch.uint8, (lib.trf_band_split_packed_bytes(_dins(dins), F),))
    _need(X, "X", torch.float32, (n_frames * F, DIM))
    _check(lib.trf_band_split(feats.data_ptr(), n_frames, F, _dins(dins), packed.data_ptr(), X.data_ptr(), _stream()))


# ---------------------------------------------------------------------------------------------- song assembly


def check_chunk_starts(starts, nc: int, L: int, n: int) -> list[int]:
    """The chunk starts of one overlap-add batch as a list of ints, after checking on the host that there
    are ``nc`` of them, strictly ascending, each chunk's ``L`` samples inside the ``n``-sample song (the
    kernel finds a sample's chunks by binary search over them).  Raises ValueError."""
    if isinstance(starts, torch.Tensor):
        if starts.is_cuda:
            raise ValueError("starts must be on the host (they are checked before upload)")
        starts = starts.tolist()
    starts = [int(s) for s in starts]
    if len(starts) != nc:
        raise ValueError(f"starts has {len(starts)} entries for {nc} chunks")
    if any(b <= a for a, b in zip(starts, starts[1:])):
        raise ValueError(f"chunk starts must be strictly ascending, got {starts}")
    if starts and (starts[0] < 0 or starts[-1] + L > n):
        raise ValueError(f"chunks must lie inside the {n}-sample song (starts {starts[0]}..{starts[-1]}, L = {L})")
    return starts


def overlap_add(y: torch.Tensor, L: int, starts, window: torch.Tensor, acc: torch.Tensor,
                wsum: torch.Tensor) -> None:
    """acc [2, n] += y[c, :, :L] * window[:L] at starts[c], wsum [n] += window[:L], chunk by chunk in
    ascending order with the reference's fp32 roundings (chunking.py:39-61). y [nc, 2, Ly] fp32.

    ``starts``: the chunks' first samples, a host sequence of ints (or a CPU int tensor).  They are checked
    here, where they can be read, to be strictly ascending with every chunk's L samples inside the song,
    then uploaded."""
    lib = load()
    nc = y.shape[0]
    _need(y, "y", torch.float32)
    if y.dim() != 3 or y.shape[1] != 2 or not 1 <= L <= y.shape[2]:
        raise ValueError(f"y must be [chunks, 2, >= L], got {tuple(y.shape)} with L = {L}")
    _need(window, "window", torch.float32)
    if window.numel() < L:
        raise ValueError("window is shorter than L")
    _need(acc, "acc", torch.float32)
    n = acc.shape[1]
    _need(acc, "acc", torch.float32, (2, n))
    _need(wsum, "wsum", torch.float32, (n,))
    sd = torch.tensor(check_chunk_starts(starts, nc, L, n), dtype=torch.int64).to(acc.device)
    _check(lib.trf_overlap_add(y.data_ptr(), nc, y.shape[2], L, sd.data_ptr(), window.data_ptr(), n,
                               acc.data_ptr(), wsum.data_ptr(), _stream()))


def overlap_finish(acc: torch.Tensor, wsum: torch.Tensor, gain: float, out: torch.Tensor) -> None:
    """out [2, n] = acc / max(wsum, 1e-10) / gain, correctly rounded (out may be acc)."""
    lib = load()
    n = acc.shape[1]
    _need(acc, "acc", torch.float32, (2, n))
    _need(wsum, "wsum", torch.float32, (n,))
    _need(out, "out", torch.float32, (2, n))
    _check(lib.trf_overlap_finish(acc.data_ptr(), wsum.data_ptr(), n, float(gain), out.data_ptr(), _stream()))
