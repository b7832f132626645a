"""ctypes binding of libtagi_hip.so (the C ABI declared in include/tagi_hip.h).

The library is loaded lazily on first use, after torch has loaded its HIP runtime, so
both share one runtime (the library's DT_NEEDED soname resolves to the copy torch
already mapped). There is no fallback: if the library or a GPU is missing, every
kernel call raises.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_uint64, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("TAGI_HIP_LIB", Path(__file__).resolve().parent / "libtagi_hip.so"))

TAGI_OK = 0
FAMILIES = [
    "conv_fwd", "conv_bwd_delta", "conv_wgrad", "linear_fwd", "linear_bwd_delta",
    "linear_wgrad", "bmm_fwd", "bmm_shared", "relu", "remax", "bn_stats", "bn_fwd",
    "bn_bwd", "update", "innovation", "add", "avgpool", "jacobian", "rmsnorm",
    "embedding", "pe", "splitk_reduce", "maxpool", "layernorm", "softplus", "attn_scores",
]
FAM_COUNT = len(FAMILIES)


class TagiView(ctypes.Structure):
    """tagi_view: element (z, i, j) at (z/zdiv)*sz1 + (z%zdiv)*sz2 + i*si + j*sj."""

    _fields_ = [("zdiv", c_int64), ("sz1", c_int64), ("sz2", c_int64), ("si", c_int64), ("sj", c_int64)]


class ConvGeom(ctypes.Structure):
    """tagi_conv_geom."""

    _fields_ = [
        (n, c_int64)
        for n in ("N", "C", "H", "W", "Cout", "k", "stride", "pad_top", "pad_left", "Ho", "Wo")
    ]


P = c_void_p
I64 = c_int64
F = c_float
class BnPending(ctypes.Structure):
    """tagi_bn_bwd_pending: one BatchNorm2D layer whose parameter deltas are still to form."""

    _fields_ = [(n, c_void_p) for n in ("ws", "Sg", "Sb", "dmg", "dSg", "dmb", "dSb")] + [
        (n, c_int64) for n in ("N", "C", "HW")
    ] + [(n, c_void_p) for n in ("cSb", "cdmb", "cdSb")] + [("nblk", c_int64)]


VP = POINTER(TagiView)
GP = POINTER(ConvGeom)
BP = POINTER(BnPending)

# name -> (restype, argtypes)
_SIGS = {
    "tagi_abi_version": (c_int, []),
    "tagi_last_error": (c_char_p, []),
    "tagi_prof_begin": (c_int, [c_uint64]),
    "tagi_stream_wait": (c_int, [P, P]),
    "tagi_prof_end": (c_int, [P, P, P, P]),
    "tagi_probe_mfma_loop": (c_int, [P, I64, I64, P]),
    "tagi_probe_mfma_mix": (c_int, [P, I64, I64, c_int, c_int, P]),
    "tagi_probe_stream": (c_int, [P, P, I64, I64, c_int, P]),
    "tagi_probe_stream_variant": (c_int, [P, P, I64, I64, I64, c_int, c_int, c_int, P]),
    "tagi_linear_fwd": (c_int, [P, P, P, P, P, P, P, P, I64, I64, I64, P, I64, P]),
    "tagi_linear_fwd_relu": (c_int, [P, P, P, P, P, P, P, P, P, I64, I64, I64, P, I64, P]),
    "tagi_linear_fwd_ws_bytes": (I64, [I64, I64, I64]),
    "tagi_linear_fwd_noalloc": (c_int, [P, P, P, P, P, P, P, P, I64, I64, I64, P]),
    "tagi_linear_bwd_delta": (c_int, [P, P, P, P, P, I64, I64, I64, P, I64, P]),
    "tagi_linear_bwd_delta_jacobian": (c_int, [P, P, P, P, P, P, I64, I64, I64, P, I64, P]),
    "tagi_linear_bwd_delta_ws_bytes": (I64, [I64, I64, I64]),
    "tagi_linear_bwd_delta_add": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, P, I64, P]),
    "tagi_linear_wgrad": (c_int, [P, P, P, P, P, P, P, P, P, I64, I64, I64, P, I64, P]),
    "tagi_linear_wgrad_update": (c_int, [P, P, P, P, P, P, P, P, P, P, P, F, I64, I64, I64, P, I64, P]),
    "tagi_linear_wgrad_ws_bytes": (I64, [I64, I64, I64]),
    "tagi_bmm_tagi": (c_int, [P, P, P, P, P, P, I64, I64, I64, I64, VP, VP, VP, F, F, P]),
    "tagi_attn_scores_remax": (c_int, [P, P, P, P, I64, P, P, P, I64, I64, I64, I64, F, F, P]),
    "tagi_attn_fwd": (c_int, [P, P, P, P, P, P, I64, P, P, P, P, P, I64, I64, I64, I64, I64, F, F, P]),
    "tagi_attn_score_deltas_qk": (c_int, [P, P, I64, P, P, I64, P, P, P, I64, I64, I64, I64, I64, F, F, c_int, P]),
    "tagi_attn_score_deltas_qk_joint": (c_int, [P, P, I64, P, P, P, I64, P, P, P, P, P, I64, I64, I64, I64, I64, F,
                                                F, P]),
    "tagi_bmm_shared": (c_int, [P, P, P, P, P, I64, I64, I64, I64, VP, VP, VP, F, F, c_int, P]),
    "tagi_bmm_shared_jacobian": (c_int, [P, P, P, P, P, P, I64, I64, I64, I64, VP, VP, VP, F, F, c_int, P]),
    "tagi_conv2d_fwd": (c_int, [P, P, P, P, P, P, P, P, GP, P, I64, P]),
    "tagi_conv2d_fwd_ws_bytes": (I64, [GP]),
    "tagi_conv2d_fwd_relu_bn_stats": (c_int, [P, P, P, P, P, P, P, P, GP, P, P, P, P, P, P, F, F, c_int, c_int, P,
                                              I64, P]),
    "tagi_conv2d_fwd_relu_bn_stats_ws_bytes": (I64, [GP]),
    "tagi_conv2d_bwd_delta": (c_int, [P, P, P, P, P, GP, P, I64, P]),
    "tagi_conv2d_bwd_delta_ws_bytes": (I64, [GP]),
    "tagi_conv2d_bwd_delta_add": (c_int, [P, P, P, P, P, P, P, GP, P, I64, P]),
    "tagi_conv2d_bwd_delta_bn_relu": (c_int, [P, P, P, P, P, P, P, F, P, P, P, I64, GP, P, I64, P]),
    "tagi_conv2d_bwd_delta_bn_relu_part_bytes": (I64, [GP]),
    "tagi_conv2d_bwd_delta_add_bn_relu": (c_int, [P, P, P, P, P, P, P, P, P, P, P, F, P, P, P, I64, GP, P, I64, P]),
    "tagi_conv2d_wgrad": (c_int, [P, P, P, P, P, P, P, P, P, GP, P, I64, P]),
    "tagi_conv2d_wgrad_ws_bytes": (I64, [GP]),
    "tagi_relu_fwd": (c_int, [P, P, P, P, P, I64, P]),
    "tagi_jacobian_bwd": (c_int, [P, P, P, P, P, I64, P]),
    "tagi_remax_fwd": (c_int, [P, P, P, P, P, I64, I64, P]),
    "tagi_innovation": (c_int, [P, P, P, F, P, P, I64, P]),
    "tagi_capped_update": (c_int, [P, P, P, P, F, I64, P]),
    "tagi_capped_update_multi": (c_int, [P, P, P, P, P, I64, F, P]),
    "tagi_add_inplace": (c_int, [P, P, P, P, I64, P]),
    "tagi_avgpool2d_fwd": (c_int, [P, P, P, P, I64, I64, I64, I64, I64, F, P]),
    "tagi_avgpool2d_bwd": (c_int, [P, P, P, P, I64, I64, I64, I64, I64, F, P]),
    "tagi_relu_avgpool2d_fwd": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, F, c_int, P]),
    "tagi_avgpool2d_relu_bwd": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, F, c_int, P]),
    "tagi_bn_stats": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, F, F, c_int, c_int, P, I64, P]),
    "tagi_bn_stats_ws_bytes": (I64, [I64, I64, I64]),
    "tagi_bn_fwd": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, F, P]),
    "tagi_bn_bwd": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, F, P, I64, P]),
    "tagi_bn_bwd_ws_bytes": (I64, [I64, I64, I64]),
    "tagi_relu_bn_stats": (c_int, [P, P, P, P, P, P, P, P, I64, I64, I64, F, F, c_int, c_int, P, I64, P]),
    "tagi_relu_bn_fwd": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, F, P]),
    "tagi_bn_relu_bwd": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, F, P, I64, P]),
    "tagi_bn_relu_bwd_partials": (c_int, [P, P, P, P, P, P, P, P, I64, I64, I64, F, P, I64, P]),
    "tagi_bn_relu_bwd_partials_bias": (c_int, [P, P, P, P, P, P, P, P, I64, I64, I64, F, P, I64, P]),
    "tagi_bn_relu_bwd_bias_ws_bytes": (I64, [I64, I64, I64]),
    "tagi_bn_bwd_finalize_multi": (c_int, [BP, I64, P]),
    "tagi_rmsnorm_fwd": (c_int, [P, P, P, P, P, P, P, I64, I64, F, P]),
    "tagi_rmsnorm_bwd": (c_int, [P, P, P, P, P, P, P, P, P, P, I64, I64, P, I64, P]),
    "tagi_rmsnorm_bwd_ws_bytes": (I64, [I64, I64]),
    "tagi_embedding_fwd": (c_int, [P, P, P, P, P, I64, I64, I64, I64, P]),
    "tagi_embedding_bwd": (c_int, [P, P, P, P, P, P, I64, I64, I64, I64, P, I64, P]),
    "tagi_embedding_bwd_ws_bytes": (I64, [I64, I64, I64]),
    "tagi_pe_add": (c_int, [P, P, P, I64, I64, I64, P]),
    "tagi_innovation_indexed": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, P]),
    "tagi_hrc_innovation": (c_int, [P, P, P, P, P, F, P, P, I64, I64, I64, I64, P]),
    "tagi_hrc_class_probs": (c_int, [P, P, P, P, F, P, P, I64, I64, I64, I64, P]),
    "tagi_innovation_heteros": (c_int, [P, P, P, P, P, I64, P]),
    "tagi_even_softplus_fwd": (c_int, [P, P, P, P, P, I64, P]),
    "tagi_maxpool2d_fwd": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, c_int, P]),
    "tagi_maxpool2d_bwd": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, c_int, P]),
    "tagi_layernorm_fwd": (c_int, [P, P, P, P, P, P, P, P, P, P, I64, I64, F, P]),
    "tagi_layernorm_bwd": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, F, P, I64, P]),
    "tagi_layernorm_bwd_ws_bytes": (I64, [I64, I64]),
}

EXPORTED = tuple(_SIGS)

_lib: ctypes.CDLL | None = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load the library (once) and declare every entry point's signature."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"libtagi_hip.so not found at {p}; build it with `python triton-tagi_amd/build.py`"
        )
    lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    msg = load().tagi_last_error()
    return msg.decode() if msg else ""


_fns: dict = {}  # (library handle id, name) -> bound entry point


def _fn(name: str):
    lib = load()
    key = (id(lib), name)
    f = _fns.get(key)
    if f is None:
        f = _fns[key] = getattr(lib, name)
    return f


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point; raise RuntimeError on failure."""
    rc = _fn(name)(*args)
    if rc != TAGI_OK:
        raise RuntimeError(f"{name} failed (status {rc}): {last_error()}")


_queries: dict = {}


def query(name: str, *args) -> int:
    """Value of a size query. Queries taking only integers (the workspace sizes of a shape,
    fixed by the deterministic plan choice) are answered once per argument tuple."""
    if all(type(a) is int for a in args):
        key = (name, *args)
        v = _queries.get(key)
        if v is None:
            v = _queries[key] = int(_fn(name)(*args))
        return v
    return int(_fn(name)(*args))


# ---------------------------------------------------------------------------------
# Tensor plumbing
# ---------------------------------------------------------------------------------
# torch's current-stream handle without building a Stream object (the public call below
# costs a few microseconds, a launch-bound step makes about 15 of them)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on t's device (the stream kernels are queued on)."""
    if _raw_stream is not None and t.is_cuda:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def stream_wait(waiter: torch.cuda.Stream, producer: torch.cuda.Stream) -> None:
    """Work queued on ``waiter`` from now on starts after the work queued on ``producer``
    so far (torch.cuda.Stream.wait_stream without the event's system-scope fence)."""
    call("tagi_stream_wait", waiter.cuda_stream, producer.cuda_stream)


def check(t: torch.Tensor, name: str, contiguous: bool = True) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype is not torch.float32:
        raise TypeError(f"{name}: expected float32, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(
            f"{name}: tensor is on {t.device}; the TAGI HIP kernels run on the GPU only"
        )
    if contiguous and not (t.is_contiguous() or (t.dim() == 4 and t.is_contiguous(memory_format=torch.channels_last))):
        raise ValueError(f"{name}: tensor must be dense (contiguous or channels-last)")
    return t


def dense(t: torch.Tensor) -> torch.Tensor:
    """t itself when its storage is dense in its own dim order (row-major or channels-last)."""
    if t.is_contiguous() or (t.dim() == 4 and t.is_contiguous(memory_format=torch.channels_last)):
        return t
    return t.contiguous()


def channels_last(t: torch.Tensor) -> torch.Tensor:
    """4-D tensor in channels-last storage (a copy only when it is not already)."""
    if t.is_contiguous(memory_format=torch.channels_last):
        return t
    return t.contiguous(memory_format=torch.channels_last)


def like(t: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """t with the same storage order as ref (elementwise kernels walk raw storage)."""
    t = dense(t)
    if t.stride() == ref.stride():
        return t
    if ref.dim() == 4 and ref.is_contiguous(memory_format=torch.channels_last):
        return t.contiguous(memory_format=torch.channels_last)
    return t.contiguous()


def empty_cl(N: int, C: int, H: int, W: int, device) -> torch.Tensor:
    return torch.empty((N, C, H, W), device=device, dtype=torch.float32, memory_format=torch.channels_last)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    """Scratch buffer from torch's caching allocator (the library never allocates)."""
    if nbytes <= 0:
        return None
    return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)


def ws_args(ws: torch.Tensor | None) -> tuple[int | None, int]:
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel() * 4)


def view(zdiv: int, sz1: int, sz2: int, si: int, sj: int) -> TagiView:
    return TagiView(int(max(zdiv, 1)), int(sz1), int(sz2), int(si), int(sj))


# ---------------------------------------------------------------------------------
# Live kernel-family timer
# ---------------------------------------------------------------------------------
def prof_begin(families: list[str] | None = None) -> None:
    mask = 0
    for i, f in enumerate(FAMILIES):
        if families is None or f in families:
            mask |= 1 << i
    call("tagi_prof_begin", mask)


def prof_end() -> dict[str, dict[str, float]]:
    ms = (ctypes.c_double * FAM_COUNT)()
    n = (ctypes.c_int64 * FAM_COUNT)()
    fl = (ctypes.c_double * FAM_COUNT)()
    by = (ctypes.c_double * FAM_COUNT)()
    call("tagi_prof_end", ctypes.addressof(ms), ctypes.addressof(n), ctypes.addressof(fl), ctypes.addressof(by))
    out = {}
    for i, f in enumerate(FAMILIES):
        if n[i]:
            out[f] = {"ms": ms[i], "launches": int(n[i]), "flops": fl[i], "bytes": by[i]}
    return out
