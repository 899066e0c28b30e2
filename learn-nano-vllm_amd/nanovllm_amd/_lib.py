"""ctypes binding of libnvk.so, the C ABI declared in include/nvk.h.

The library is HIP code built for gfx950 and has no PyTorch dependency; this
module only turns torch tensors into device pointers, element strides and the
current HIP stream.  There is deliberately no CPU path: every entry point
raises if the library is missing or a tensor is not on a GPU.

Load order matters: ``import torch`` first loads torch's copy of
libamdhip64.so.7; libnvk.so names the same SONAME, so the dynamic linker
binds it to that already-loaded HIP runtime and torch's stream handles are
valid inside the library.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnvk.so")

NVK_DTYPE_BF16 = 0
NVK_DTYPE_F16 = 1
NVK_DTYPE_F32 = 2

# Every symbol include/nvk.h declares, with its ctypes signature.
_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_ptr = ctypes.c_void_p
SIGNATURES = {
    "nvk_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "nvk_build_target": (ctypes.c_char_p, []),
    "nvk_kv_store": (ctypes.c_int, [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_i64,
                                    _c_i32, _c_i32, _c_i64, _c_ptr]),
    "nvk_paged_decode": (ctypes.c_int, [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_i64,
                                        _c_ptr, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                        _c_i32, ctypes.c_float, _c_ptr, _c_i64, _c_i64, _c_ptr,
                                        ctypes.c_size_t, _c_i32, _c_ptr]),
    "nvk_paged_decode_workspace_size": (ctypes.c_size_t,
                                        [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "nvk_paged_decode_noalloc": (ctypes.c_int, [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr,
                                                _c_i64, _c_ptr, _c_i32, _c_i32, _c_i32, _c_i32,
                                                _c_i32, _c_i32, _c_i32, ctypes.c_float, _c_ptr,
                                                _c_i64, _c_i64, _c_i32, _c_ptr]),
    "nvk_paged_decode_noalloc_init": (ctypes.c_int, []),
    "nvk_varlen_prefill": (ctypes.c_int, [_c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64,
                                          _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i32, _c_i32,
                                          _c_i32, _c_ptr, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                          _c_i32, _c_i32, ctypes.c_float, _c_ptr, _c_i64, _c_i64,
                                          _c_ptr, ctypes.c_size_t, _c_i32, _c_ptr]),
    "nvk_varlen_prefill_workspace_size": (ctypes.c_size_t,
                                          [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "nvk_prefill_tile_order_size": (ctypes.c_size_t, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                                      _c_i32]),
    "nvk_prefill_tile_order": (ctypes.c_int, [_c_ptr, _c_ptr, _c_i32, _c_i32, _c_i32, _c_i32,
                                              _c_i32, _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr]),
    "nvk_varlen_prefill_ordered": (ctypes.c_int, [_c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
                                                  _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
                                                  _c_i32, _c_i32, _c_i32, _c_ptr, _c_i64, _c_i32,
                                                  _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                                  ctypes.c_float, _c_ptr, _c_i64, _c_i64, _c_ptr,
                                                  ctypes.c_size_t, _c_ptr, ctypes.c_size_t, _c_i32,
                                                  _c_ptr]),
    "nvk_qk_norm_rope_store": (ctypes.c_int, [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr,
                                              ctypes.c_float, _c_ptr, _c_i64, _c_i64, _c_i32,
                                              _c_i32, _c_i32, _c_ptr, _c_i64, _c_i64, _c_ptr,
                                              _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_i64,
                                              _c_i32, _c_ptr]),
    "nvk_paged_decode_prologue": (ctypes.c_int, [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr,
                                                 ctypes.c_float, _c_ptr, _c_i64, _c_i64, _c_ptr,
                                                 _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr,
                                                 _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                                 _c_i32, ctypes.c_float, _c_ptr, _c_i64, _c_i64,
                                                 _c_ptr, ctypes.c_size_t, _c_i32, _c_ptr]),
    "nvk_prefill_metadata": (ctypes.c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i32, _c_i32, _c_i32,
                                            _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                            _c_ptr]),
    "nvk_decode_metadata": (ctypes.c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i32, _c_i32, _c_i32, _c_i32,
                                           _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr]),
    "nvk_decode_graph_refresh": (ctypes.c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i32,
                                                _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64,
                                                _c_i32, _c_ptr]),
    "nvk_uniform_cu_seqlens": (ctypes.c_int, [_c_ptr, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr]),
    "nvk_sample_workspace_size": (ctypes.c_size_t, [_c_i32, _c_i32]),
    "nvk_sample": (ctypes.c_int, [_c_ptr, _c_i64, _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_i64,
                                  ctypes.c_uint64, ctypes.c_uint64, _c_ptr, _c_ptr, ctypes.c_size_t,
                                  _c_ptr]),
    "nvk_gather_last_tokens": (ctypes.c_int, [_c_ptr, _c_i64, _c_ptr, _c_i32, _c_i32, _c_i32, _c_ptr,
                                              _c_i64, _c_ptr]),
}

_lib: ctypes.CDLL | None = None


class NvkError(RuntimeError):
    """A call into libnvk.so was rejected or its launch failed."""


def load() -> ctypes.CDLL:
    """Load libnvk.so once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NvkError(f"{LIB_PATH} is not built; run `make -C learn-nano-vllm_amd` "
                           "or __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(code: int) -> None:
    if code != 0:
        msg = load().nvk_strerror(code).decode()
        raise NvkError(f"nvk error {code}: {msg}")


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return NVK_DTYPE_BF16
    if t.dtype == torch.float16:
        return NVK_DTYPE_F16
    if t.dtype == torch.float32:
        return NVK_DTYPE_F32
    raise NvkError(f"unsupported dtype {t.dtype}")


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one GPU; returns that device (no CPU fallback exists)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise NvkError("nanovllm_amd kernels run on the GPU only; got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise NvkError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise NvkError("no tensor given")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# Workspaces of the attention wrappers.
#
# Eager calls: one buffer per (device, stream), grown on demand.  Calls on one
# stream run one after the other, so they can share it (every kernel writes
# what it reads in the same call).  A buffer a larger one replaces is simply
# dropped: torch's allocator returns it to the pool of the stream it was
# allocated on, which only hands it out again to work ordered after the calls
# that used it.
#
# Calls under graph capture: a fresh buffer per call, never cached.  It comes
# from the graph's private memory pool, so it lives as long as the graph and
# is never shared with eager calls, whatever stream handle torch later hands
# out again (a replay may run beside eager work on another stream).  Graphs
# that share one pool share its memory, as torch's own captured tensors do:
# replay them one at a time, as the reference's bucketed decode graphs are.
_workspaces: dict = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A uint8 device buffer of at least nbytes for the current stream of
    `device` (None for 0 bytes); torch's allocator hands out 512-byte aligned
    blocks."""
    if nbytes <= 0:
        return None
    with torch.cuda.device(device):
        if torch.cuda.is_current_stream_capturing():
            return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf
