"""ctypes binding of libbzgemv.so (the C ABI declared in include/bz_gemv.h and
include/bz_attn.h).

torch is imported before the library is opened: both link the HIP runtime by
its SONAME (libamdhip64.so.7), so the library binds to the runtime torch has
already loaded and the hipStream_t / device pointers torch hands out are valid
in it.  There is no fallback: if the library is missing the import fails.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = Path(os.environ.get("BZ_LIB", str(Path(__file__).resolve().parent / "libbzgemv.so")))
ABI_VERSION = 4

# enums of include/bz_gemv.h
OK = 0
ERR_INVALID_ARG, ERR_SHAPE, ERR_ALIGNMENT, ERR_UNSUPPORTED, ERR_LAUNCH, ERR_ABI, ERR_SCRATCH = 1, 2, 3, 4, 5, 6, 7
GEMV_SCRATCH_BYTES = 8 << 20  # BZ_GEMV_SCRATCH_BYTES
W_INT4_ZP, W_INT4_MIN, W_FP8, W_BF16 = 0, 1, 2, 3
W_INT4_TILED, W_INT4_TILED_PAIRED, W_FP8_TILED, W_FP8_TILED_PAIRED = 4, 5, 6, 7
EPI_NONE, EPI_SILU_GATE, EPI_RESIDUAL = 0, 1, 2
DT_BF16, DT_F32 = 0, 1
MASK_BOOL = 2  # include/bz_attn.h

EXPORTS = (
    "bz_abi_version",
    "bz_strerror",
    "bz_stream_capture",
    "bz_gemv_workspace",
    "bz_gemv",
    "bz_gemv_noalloc",
    "bz_rmsnorm",
    "bz_silu_mul",
    "bz_quantize_int4",
    "bz_quantize_fp8",
    "bz_dequant",
    "bz_tiled_bytes",
    "bz_pack_tiled",
    "bz_head_f32",
    "bz_qkv_rope_cache",
    "bz_attn_decode",
    "bz_attn_step",
    "bz_attn_workspace",
    "bz_attn_default_split",
    "bz_sample_cfg",
    "bz_stream_read",
    "bz_shared_read",
)


class GemvDesc(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("M", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("group", ctypes.c_int32),
        ("wfmt", ctypes.c_int32),
        ("epilogue", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("residual_dtype", ctypes.c_int32),
        ("cfg_depth", ctypes.c_int32),
        ("cfg_waves", ctypes.c_int32),
        ("cfg_tiles", ctypes.c_int32),
        ("cfg_path", ctypes.c_int32),
        ("cfg_slices", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("x", ctypes.c_void_p),
        ("ldx", ctypes.c_int64),
        ("w", ctypes.c_void_p),
        ("sc0", ctypes.c_void_p),
        ("sc1", ctypes.c_void_p),
        ("gamma", ctypes.c_void_p),
        ("residual", ctypes.c_void_p),
        ("ldr", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("ldo", ctypes.c_int64),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("out2", ctypes.c_void_p),
        ("ldo2", ctypes.c_int64),
        ("n_out2", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
    ]


class BzError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} (status {status})")


_lib: ctypes.CDLL | None = None


def _declare(lib: ctypes.CDLL) -> None:
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    lib.bz_abi_version.restype = ctypes.c_int
    lib.bz_abi_version.argtypes = []
    lib.bz_strerror.restype = ctypes.c_char_p
    lib.bz_strerror.argtypes = [ctypes.c_int]
    lib.bz_stream_capture.restype = ctypes.c_int
    lib.bz_stream_capture.argtypes = [vp, ctypes.POINTER(i32), ctypes.POINTER(ctypes.c_uint64)]
    lib.bz_gemv_workspace.restype = ctypes.c_size_t
    lib.bz_gemv_workspace.argtypes = [ctypes.POINTER(GemvDesc)]
    lib.bz_gemv.restype = ctypes.c_int
    lib.bz_gemv.argtypes = [ctypes.POINTER(GemvDesc), vp]
    lib.bz_gemv_noalloc.restype = ctypes.c_int
    lib.bz_gemv_noalloc.argtypes = [ctypes.POINTER(GemvDesc), vp]
    lib.bz_rmsnorm.restype = ctypes.c_int
    lib.bz_rmsnorm.argtypes = [vp, i64, vp, f32, vp, i64, i32, i32, vp]
    lib.bz_silu_mul.restype = ctypes.c_int
    lib.bz_silu_mul.argtypes = [vp, i64, vp, i64, vp, i64, i32, i32, vp]
    lib.bz_quantize_int4.restype = ctypes.c_int
    lib.bz_quantize_int4.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp]
    lib.bz_quantize_fp8.restype = ctypes.c_int
    lib.bz_quantize_fp8.argtypes = [vp, i32, i32, i32, f32, vp, vp, vp]
    lib.bz_dequant.restype = ctypes.c_int
    lib.bz_dequant.argtypes = [i32, vp, vp, vp, i32, i32, i32, vp, vp]
    lib.bz_tiled_bytes.restype = ctypes.c_size_t
    lib.bz_tiled_bytes.argtypes = [i32, i32, i32]
    lib.bz_pack_tiled.restype = ctypes.c_int
    lib.bz_pack_tiled.argtypes = [i32, vp, vp, i32, i32, i32, i32, vp, i32, i32, vp]
    lib.bz_head_f32.restype = ctypes.c_int
    lib.bz_head_f32.argtypes = [vp, i64, i32, i32, vp, i32, i64, i32, vp, i64, vp, i64, vp]
    lib.bz_qkv_rope_cache.restype = ctypes.c_int
    lib.bz_qkv_rope_cache.argtypes = [vp, i64, i32, i32, i32, i32, vp, vp, f32, vp, vp, i32, i64, vp, vp, vp, vp,
                                      i32, i32, vp, vp]
    lib.bz_attn_decode.restype = ctypes.c_int
    lib.bz_attn_decode.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, i32, i64, vp, f32, i32, vp, vp, i64,
                                   vp]
    lib.bz_attn_step.restype = ctypes.c_int
    lib.bz_attn_step.argtypes = [vp, i64, i32, i32, i32, i32, vp, vp, f32, vp, vp, i32, i64, vp, vp, vp, i32, i32, vp,
                                 vp, i32, i64, f32, i32, vp, vp, i64, vp]
    lib.bz_attn_workspace.restype = ctypes.c_size_t
    lib.bz_attn_workspace.argtypes = [i32, i32, i32, i32, i32]
    lib.bz_attn_default_split.restype = ctypes.c_int32
    lib.bz_attn_default_split.argtypes = [i32]
    lib.bz_stream_read.restype = ctypes.c_int
    lib.bz_stream_read.argtypes = [vp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_uint32, vp, vp]
    lib.bz_shared_read.restype = ctypes.c_int
    lib.bz_shared_read.argtypes = [vp, ctypes.c_size_t, vp, ctypes.c_size_t, i32, ctypes.c_uint32, vp, vp]
    lib.bz_sample_cfg.restype = ctypes.c_int
    lib.bz_sample_cfg.argtypes = [vp, i64, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m breeze_amd.build` "
                "(the GPU path has no fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        _declare(handle)
        version = handle.bz_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {version}, this binding expects {ABI_VERSION}")
        _lib = handle
    return _lib


def strerror(status: int) -> str:
    try:
        return lib().bz_strerror(status).decode()
    except Exception:  # noqa: BLE001 - only used to format an error
        return "unknown"


def check(status: int, what: str) -> None:
    if status != OK:
        raise BzError(status, what)


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def capture_of(stream: int):
    """The id of the graph capture under way on the raw HIP stream, or None."""
    active, cid = ctypes.c_int32(0), ctypes.c_uint64(0)
    check(lib().bz_stream_capture(stream, ctypes.byref(active), ctypes.byref(cid)), "bz_stream_capture")
    return cid.value if active.value else None


def stream_workspace(table: dict, key: tuple, nbytes: int, device: torch.device, stream: int,
                     retired: list) -> torch.Tensor:
    """A zero-filled int32 buffer of at least ``nbytes`` owned by
    (``key``, stream) -- and, while a graph capture is under way on the
    stream, by that capture -- so calls on different streams, and different
    captured graphs, never share one.

    Outside a capture the buffer is allocated and zeroed eagerly on the
    stream.  Inside a capture it comes from the graph's memory pool and its
    zero fill (a fill kernel, not a memset node) is recorded into the graph,
    ahead of the calls that use it, so every replay starts from zeroed
    counters; the kernels leave them zero again either way.  An outgrown
    buffer is kept in ``retired`` for the life of the process, since a graph
    captured earlier may still point at it."""
    cap = capture_of(stream)
    full = key + (stream, cap)
    buf = table.get(full)
    if buf is None or buf.numel() * 4 < nbytes:
        n = max(nbytes, 2 * (buf.numel() * 4 if buf is not None else 0), 1 << 20)
        if buf is not None:
            retired.append(buf)
        buf = torch.zeros(-(-n // 4), dtype=torch.int32, device=device)
        table[full] = buf
    return buf
