"""Loading of the in-tree native libraries. There is no fallback: a missing library is an error."""

import ctypes
import re
from pathlib import Path

import torch

PKG = Path(__file__).resolve().parent
LIB_DIR = PKG / "lib"
CABI_PATH = LIB_DIR / "libie_attn.so"
TORCH_OPS_PATH = LIB_DIR / "_ie_torch_ops.so"
HEADER = PKG.parent / "include" / "ie_attn.h"

_ops_loaded = False
_cabi = None


class NativeLibraryMissing(RuntimeError):
    pass


def _require(path: Path) -> None:
    if not path.exists():
        raise NativeLibraryMissing(
            f"{path} is not built; run `python __graft_entry__.py` (build()) or "
            f"`python {PKG.name}/build.py` first")


def ops():
    """torch.ops.ie, loading lib/_ie_torch_ops.so on first use."""
    global _ops_loaded
    if not _ops_loaded:
        _require(CABI_PATH)
        _require(TORCH_OPS_PATH)
        torch.ops.load_library(str(TORCH_OPS_PATH))
        _ops_loaded = True
    return torch.ops.ie


def cabi() -> ctypes.CDLL:
    """libie_attn.so through ctypes (the C ABI of include/ie_attn.h)."""
    global _cabi
    if _cabi is None:
        _require(CABI_PATH)
        _cabi = ctypes.CDLL(str(CABI_PATH))
        _cabi.ie_attn_version.restype = ctypes.c_int32
        _cabi.ie_attn_last_error.restype = ctypes.c_char_p
        _cabi.ie_decode_attention_workspace_size.restype = ctypes.c_size_t
        _cabi.ie_decode_attention_workspace_size.argtypes = [ctypes.c_int32] * 3
        _cabi.ie_decode_attention_max_splits.restype = ctypes.c_int32
        _cabi.ie_decode_attention_max_splits.argtypes = [ctypes.c_int32]
        _cabi.ie_decode_attention_target.restype = ctypes.c_int32
        _cabi.ie_decode_attention_target.argtypes = [ctypes.c_int32, ctypes.c_int32]
        _cabi.ie_decode_attention_workspace_counts_bytes.restype = ctypes.c_size_t
        _cabi.ie_decode_attention_workspace_counts_bytes.argtypes = [ctypes.c_int32] * 2
        _cabi.ie_prefill_attention_workspace_counts_bytes.restype = ctypes.c_size_t
        _cabi.ie_prefill_attention_workspace_counts_bytes.argtypes = []
        _cabi.ie_prefill_attention_grid.restype = ctypes.c_int32
        _cabi.ie_prefill_attention_grid.argtypes = [ctypes.c_int32] * 4
    return _cabi


def header_functions() -> list:
    """Names of the functions include/ie_attn.h declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ie_[a-z0-9_]+)\s*\(", text)))


class KVCacheDesc(ctypes.Structure):
    """ctypes twin of `ie_kv_cache` (include/ie_attn.h)."""

    _fields_ = [
        ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p), ("v_scale", ctypes.c_void_p),
        ("k_calibration", ctypes.c_void_p),
        ("pool", ctypes.c_int64), ("num_kv_heads", ctypes.c_int64),
        ("max_len", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("stride_slot", ctypes.c_int64), ("stride_head", ctypes.c_int64),
        ("stride_tok", ctypes.c_int64),
        ("scale_stride_slot", ctypes.c_int64), ("scale_stride_head", ctypes.c_int64),
        ("cal_stride_slot", ctypes.c_int64), ("cal_stride_head", ctypes.c_int64),
    ]

    @staticmethod
    def of(cache) -> "KVCacheDesc":
        k = cache.k
        return KVCacheDesc(
            k.data_ptr(), cache.v.data_ptr(), cache.k_scale.data_ptr(), cache.v_scale.data_ptr(),
            cache.k_calibration.data_ptr(), k.shape[0], k.shape[1], k.shape[2], k.shape[3],
            k.stride(0), k.stride(1), k.stride(2), cache.k_scale.stride(0),
            cache.k_scale.stride(1), cache.k_calibration.stride(0),
            cache.k_calibration.stride(1))
