"""ctypes binding of the C ABI in ``include/svoo_hip.h`` (library ``svoo_amd/_svoo_hip.so``).

torch is imported first so that the library's ``libamdhip64.so.7`` dependency resolves to the HIP
runtime torch already loaded: device pointers and streams are then shared with torch.  There is no
fallback: if the library is missing or a GPU is absent, calls raise.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_longlong, c_size_t, c_void_p
from pathlib import Path
from typing import Dict, Optional

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = Path(__file__).resolve().with_name("_svoo_hip.so")

P = c_void_p
_SIGS = {
    "svoo_version": (c_int, []),
    "svoo_last_error": (ctypes.c_char_p, []),
    "svoo_cluster_sort_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "svoo_cluster_sort": (c_int, [P, c_int, c_int, c_int, P, P, P, P, P, c_size_t, P]),
    "svoo_permute_rows": (c_int, [P, P, P, c_int, c_int, c_int, c_int, P]),
    "svoo_permute_rows2": (c_int, [P, P, P, P, P, c_int, c_int, c_int, P]),
    "svoo_unpermute_rows": (c_int, [P, P, P, c_int, c_int, c_int, P]),
    "svoo_unpermute_rows_bshd": (c_int, [P, P, P, c_int, c_int, c_int, c_int, P]),
    "svoo_centroid_update_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "svoo_centroid_update": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, P, c_size_t, P]),
    "svoo_l2norm_rows": (c_int, [P, c_int, P, c_longlong, c_int, c_float, P]),
    "svoo_convert": (c_int, [P, c_int, P, c_int, c_longlong, P]),
    "svoo_convert_rows": (c_int, [P, c_int, c_int, P, c_int, c_int, c_longlong, P]),
    "svoo_cocluster_prep": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "svoo_cocluster_assign": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "svoo_co_cluster_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "svoo_co_cluster": (c_int, [P, P, c_int, c_int, c_int, c_int, c_int, c_int,
                                P, P, P, P, P, P, P, P, P, P, P, c_size_t, P]),
    "svoo_centroid_scores": (c_int, [P, P, c_int, c_int, c_int, c_int, P, P]),
    "svoo_block_mask": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, c_int, P, P, P, P]),
    "svoo_weighted_softmax": (c_int, [P, P, c_longlong, P, c_longlong, c_int, P]),
    "svoo_vbsa_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "svoo_vbsa_fwd": (c_int, [P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P, c_size_t, P, P]),
    "svoo_vbsa_segments": (c_int, [P, P, c_int, c_int, c_int, P, P, P, P]),
    "svoo_vbsa_fused_fwd": (c_int, [P, P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, P, c_size_t,
                                    P, P]),
    "svoo_vbsa_fused_fwd_noalloc": (c_int, [P, P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int,
                                            P, P]),
    "svoo_probe_mfma_layout": (c_int, [P, P, P]),
    "svoo_probe_mfma_f64_layout": (c_int, [P, P]),
    "svoo_exact_sparsity_counts": (c_int, [P, c_longlong, c_int, c_float, c_float, P, P]),
    "svoo_ear_value_stats": (c_int, [P, P, P, c_int, c_int, c_int, c_int, c_int, P, P, P, P]),
    "svoo_ear_centroid_logits": (c_int, [P, P, c_int, c_int, c_int, c_int, P, P]),
    "svoo_ear_efficiency": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, c_float,
                                    P, P]),
    "svoo_ear_select": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_float, P, P]),
    "svoo_vbsa_ear_fwd": (c_int, [P, P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P, c_size_t, P, P]),
}

EXPORTED_SYMBOLS = tuple(_SIGS)

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load the HIP library (once) and declare its signatures."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"SVOO HIP library not found at {LIB_PATH}; build it with "
                "`python -m svoo_amd.build` (or __graft_entry__.build())"
            )
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def last_error() -> str:
    msg = lib().svoo_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise ``RuntimeError`` with the library message on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed ({rc}): {last_error()}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_of(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an integer handle."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu_tensor(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise AssertionError(f"{name} must be a GPU (HIP) tensor")


_ELEM_TYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def convert(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``x`` in ``dtype`` through the HIP conversion kernel (bf16 / fp16 / fp32; rounding to nearest even)."""
    if x.dtype == dtype:
        return x
    if x.dtype not in _ELEM_TYPES or dtype not in _ELEM_TYPES:
        raise TypeError(f"the MI355X path takes bfloat16, float16 or float32 tensors, got {x.dtype} -> {dtype}")
    require_gpu_tensor(x, "x")
    xx = x.contiguous()
    out = torch.empty(xx.shape, dtype=dtype, device=xx.device)
    call("svoo_convert", xx.data_ptr(), _ELEM_TYPES[xx.dtype], out.data_ptr(), _ELEM_TYPES[dtype], xx.numel(),
         stream_of(xx.device))
    return out


def as_bf16(x: torch.Tensor, name: str) -> torch.Tensor:
    """The bf16 operand of a kernel: bf16 tensors as they are, fp16 / fp32 rounded to bf16 (to nearest even)."""
    if not isinstance(x, torch.Tensor) or x.dtype not in _ELEM_TYPES:
        raise TypeError(f"{name}: the MI355X path takes bfloat16, float16 or float32 tensors, got "
                        f"{getattr(x, 'dtype', type(x).__name__)}")
    require_gpu_tensor(x, name)
    return convert(x, torch.bfloat16)


ROW = 128  # elements per row of every kernel operand; head dims below it are zero-padded


def as_rows128(x: torch.Tensor, name: str) -> torch.Tensor:
    """``x [..., D]`` (D <= 128; bf16 / fp16 / fp32) as the kernels' bf16 operand ``[..., 128]``: fp16 / fp32 rounded
    to bf16 (to nearest even), columns past D zero."""
    if not isinstance(x, torch.Tensor) or x.dtype not in _ELEM_TYPES:
        raise TypeError(f"{name}: the MI355X path takes bfloat16, float16 or float32 tensors, got "
                        f"{getattr(x, 'dtype', type(x).__name__)}")
    d = x.shape[-1] if x.dim() else 0
    if not 1 <= d <= ROW:
        raise ValueError(f"{name}: head dim {d} (the MI355X path takes 1..{ROW})")
    if d == ROW:
        return as_bf16(x, name)
    require_gpu_tensor(x, name)
    xx = x.contiguous()
    out = torch.empty(*xx.shape[:-1], ROW, dtype=torch.bfloat16, device=xx.device)
    call("svoo_convert_rows", xx.data_ptr(), _ELEM_TYPES[xx.dtype], d, out.data_ptr(), 0, ROW, xx.numel() // d,
         stream_of(xx.device))
    return out


def from_rows128(y: torch.Tensor, d: int, dtype: torch.dtype) -> torch.Tensor:
    """Rows of 128 back to the caller's head dim ``d`` (the first d columns) and dtype."""
    if d == ROW:
        return convert(y, dtype)
    yy = y.contiguous()
    out = torch.empty(*yy.shape[:-1], d, dtype=dtype, device=yy.device)
    call("svoo_convert_rows", yy.data_ptr(), _ELEM_TYPES[yy.dtype], ROW, out.data_ptr(), _ELEM_TYPES[dtype], d,
         yy.numel() // ROW, stream_of(yy.device))
    return out


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned scratch from torch's caching allocator (no hipMalloc on the steady state)."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
