"""Loader and ctypes mirror of the C ABI in ``include/linattn_hip.h``.

The shared library ``linattn_amd/_lib/liblinattn_hip.so`` is built in-tree by
``linattn_amd.build.build()`` (hipcc, gfx950).  Like the reference's C kernel
loader (kernels/c_attention.py:37-65) the library is opened with ``ctypes``;
unlike it, nothing is compiled at import time and there is no fallback: a
missing library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "liblinattn_hip.so"
ABI_VERSION = 13

LA_F32, LA_BF16, LA_F16, LA_FP8_E4M3, LA_F64 = 0, 1, 2, 3, 4
LA_OK, LA_ERR_INVALID, LA_ERR_UNSUPPORTED, LA_ERR_HIP, LA_ERR_WORKSPACE = 0, 1, 2, 3, 4

EXPORTED = (
    "la_abi_version",
    "la_last_error",
    "la_sparse_attention_workspace",
    "la_sparse_attention",
    "la_sparse_attention_noalloc",
    "la_quest_page_bounds",
    "la_quest_scores",
    "la_quest_select",
    "la_quest_decode_fused",
    "la_topk_rows_workspace",
    "la_topk_rows",
    "la_indexer_topk_workspace",
    "la_indexer_topk",
    "la_block_select_workspace",
    "la_block_select",
    "la_block_sparse_prefill_workspace",
    "la_block_sparse_prefill",
    "la_paged_kv_append",
    "la_gate_select_workspace",
    "la_gate_select",
    "la_block_means",
    "la_xattn_select_workspace",
    "la_xattn_select",
    "la_device_status",
    "la_test_set_spin_limit",
)

LA_DEV_TOPK_TIMEOUT = 1
LA_DEV_PREFILL_RANGE = 2
NOALLOC_MAX_WORKSPACE = 16 << 20  # LA_NOALLOC_MAX_WORKSPACE

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


class LaKV(ctypes.Structure):
    _fields_ = [("k", _vp), ("v", _vp), ("k_scale", _vp), ("v_scale", _vp), ("page_table", _vp),
                ("kv_len", _vp), ("T", _i64), ("k_sb", _i64), ("k_sh", _i64), ("k_st", _i64),
                ("v_sb", _i64), ("v_sh", _i64), ("v_st", _i64), ("s_sb", _i64), ("s_sh", _i64),
                ("s_st", _i64), ("pt_stride", _i64), ("page_size", _i64), ("dtype", _i32),
                ("reserved", _i32)]


class LaSparseAttnArgs(ctypes.Structure):
    _fields_ = [("q", _vp), ("out", _vp), ("ids", _vp), ("counts", _vp), ("workspace", _vp),
                ("ws_bytes", _i64), ("B", _i64), ("Hq", _i64), ("Hkv", _i64), ("Tq", _i64),
                ("D", _i64), ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64), ("o_sb", _i64),
                ("o_sh", _i64), ("o_st", _i64), ("ids_heads", _i64), ("ids_rows", _i64),
                ("N", _i64), ("id_sb", _i64), ("id_sh", _i64), ("id_st", _i64), ("unit", _i64),
                ("offset", _i64), ("num_splits", _i64), ("scale", ctypes.c_float),
                ("q_dtype", _i32), ("out_dtype", _i32), ("causal", _i32)]


class LaTopkArgs(ctypes.Structure):
    _fields_ = [("scores", _vp), ("out_idx", _vp), ("out_val", _vp), ("out_count", _vp),
                ("n_valid", _vp), ("own", _vp), ("workspace", _vp), ("ws_bytes", _i64),
                ("B", _i64), ("H", _i64), ("Tq", _i64), ("n", _i64), ("row_stride", _i64),
                ("group", _i64), ("k", _i64), ("width", _i64), ("sink_units", _i64),
                ("window_units", _i64), ("pos_offset", _i64), ("pos_unit", _i64),
                ("force_own", _i32), ("order", _i32)]


class LaQuestSelectArgs(ctypes.Structure):
    _fields_ = [("q", _vp), ("page_min", _vp), ("page_max", _vp), ("out_idx", _vp),
                ("out_count", _vp), ("B", _i64), ("Hq", _i64), ("Hkv", _i64), ("Tq", _i64),
                ("D", _i64), ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64), ("n_pages", _i64),
                ("m_sb", _i64), ("m_sh", _i64), ("m_sp", _i64), ("m_sd", _i64),
                ("page_size", _i64), ("pos_offset", _i64), ("k", _i64), ("q_dtype", _i32),
                ("meta_dtype", _i32), ("positions", _vp)]


class LaQuestDecodeArgs(ctypes.Structure):
    _fields_ = [("select", LaQuestSelectArgs), ("kv", LaKV), ("out", _vp), ("o_sb", _i64),
                ("o_sh", _i64), ("o_st", _i64), ("scale", ctypes.c_float), ("out_dtype", _i32)]


class LaKvAppendArgs(ctypes.Structure):
    _fields_ = [("k_new", _vp), ("v_new", _vp), ("k_pool", _vp), ("v_pool", _vp),
                ("k_scale", _vp), ("v_scale", _vp), ("page_table", _vp), ("positions", _vp),
                ("page_min", _vp), ("page_max", _vp), ("B", _i64), ("Hkv", _i64), ("Tn", _i64),
                ("D", _i64), ("n_sb", _i64), ("n_sh", _i64), ("n_st", _i64), ("n_phys", _i64),
                ("pool_page", _i64), ("pt_sb", _i64), ("pt_pages", _i64), ("meta_page", _i64),
                ("n_pages", _i64), ("m_sb", _i64), ("m_sh", _i64), ("m_sp", _i64), ("m_sd", _i64),
                ("in_dtype", _i32), ("pool_dtype", _i32), ("s_stride", _i64)]


class LaIndexerArgs(ctypes.Structure):
    _fields_ = [("q", _vp), ("kk", _vp), ("w", _vp), ("out_idx", _vp), ("out_val", _vp),
                ("workspace", _vp), ("ws_bytes", _i64), ("B", _i64), ("Tq", _i64), ("Tk", _i64),
                ("HI", _i64), ("d", _i64), ("k", _i64), ("q_sb", _i64), ("q_st", _i64),
                ("q_sh", _i64), ("k_sb", _i64), ("k_st", _i64), ("k_sh", _i64), ("w_sb", _i64),
                ("w_st", _i64), ("w_sh", _i64), ("offset", _i64), ("q_chunk", _i64),
                ("causal_unit", _i64), ("in_dtype", _i32), ("causal", _i32), ("order", _i32),
                ("reserved", _i32)]


class LaBlockSelectArgs(ctypes.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("out_idx", _vp), ("out_count", _vp), ("workspace", _vp),
                ("ws_bytes", _i64), ("B", _i64), ("Hq", _i64), ("Hkv", _i64), ("T", _i64),
                ("D", _i64), ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64), ("k_sb", _i64),
                ("k_sh", _i64), ("k_st", _i64), ("block", _i64), ("topk", _i64),
                ("sink_blocks", _i64), ("window_blocks", _i64), ("width", _i64),
                ("in_dtype", _i32), ("reserved", _i32), ("lengths", _vp)]


class LaGateSelectArgs(ctypes.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("out_idx", _vp), ("out_count", _vp), ("workspace", _vp),
                ("ws_bytes", _i64), ("B", _i64), ("Hq", _i64), ("Hkv", _i64), ("Tq", _i64),
                ("T", _i64), ("D", _i64), ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64),
                ("k_sb", _i64), ("k_sh", _i64), ("k_st", _i64), ("block", _i64), ("topk", _i64),
                ("offset", _i64), ("width", _i64), ("in_dtype", _i32), ("reserved", _i32),
                ("kbar", _vp)]


class LaBlockMeansArgs(ctypes.Structure):
    _fields_ = [("k", _vp), ("out", _vp), ("positions", _vp), ("lengths", _vp), ("B", _i64),
                ("H", _i64), ("T", _i64), ("D", _i64), ("k_sb", _i64), ("k_sh", _i64),
                ("k_st", _i64), ("block", _i64), ("first_block", _i64), ("n_blocks", _i64),
                ("in_dtype", _i32), ("reserved", _i32)]


class LaXattnSelectArgs(ctypes.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("out_idx", _vp), ("out_count", _vp), ("alpha", _vp),
                ("B", _i64), ("Hq", _i64), ("Hkv", _i64), ("Tq", _i64), ("T", _i64), ("D", _i64),
                ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64), ("k_sb", _i64), ("k_sh", _i64),
                ("k_st", _i64), ("block", _i64), ("stride", _i64), ("offset", _i64),
                ("topk", _i64), ("width", _i64), ("inv_sqrt_d", ctypes.c_double),
                ("mode", _i32), ("in_dtype", _i32), ("workspace", _vp), ("ws_bytes", _i64)]


class LaPrefillArgs(ctypes.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp), ("ids", _vp), ("counts", _vp),
                ("workspace", _vp), ("ws_bytes", _i64),
                ("B", _i64), ("Hq", _i64), ("Hkv", _i64), ("T", _i64), ("D", _i64),
                ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64), ("k_sb", _i64), ("k_sh", _i64),
                ("k_st", _i64), ("v_sb", _i64), ("v_sh", _i64), ("v_st", _i64), ("o_sb", _i64),
                ("o_sh", _i64), ("o_st", _i64), ("block", _i64), ("width", _i64),
                ("scale", ctypes.c_float), ("causal", _i32), ("out_dtype", _i32),
                ("reserved", _i32), ("lengths", _vp), ("k_scale", _vp), ("v_scale", _vp),
                ("s_sb", _i64), ("s_sh", _i64), ("s_st", _i64), ("kv_dtype", _i32),
                ("reserved2", _i32)]


_LIB: Optional[ctypes.CDLL] = None


def library_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Open the HIP library (once).  Raises RuntimeError when it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(f"linattn_amd HIP library not built: {LIB_PATH} "
                           "(run `python -c 'import __graft_entry__ as g; g.build()'`)")
    L = ctypes.CDLL(str(LIB_PATH))
    L.la_abi_version.restype = ctypes.c_int
    L.la_last_error.restype = ctypes.c_char_p
    P = ctypes.POINTER
    L.la_sparse_attention_workspace.argtypes = [P(LaSparseAttnArgs), P(LaKV)]
    L.la_sparse_attention_workspace.restype = ctypes.c_size_t
    L.la_sparse_attention.argtypes = [P(LaSparseAttnArgs), P(LaKV), _vp]
    L.la_sparse_attention_noalloc.argtypes = [P(LaSparseAttnArgs), P(LaKV), _vp]
    L.la_quest_page_bounds.argtypes = [P(LaKV), _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp,
                                       _i64, _i64, _i64, _i64, _i32, _vp]
    L.la_quest_scores.argtypes = [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp,
                                  _i32, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp]
    L.la_quest_select.argtypes = [P(LaQuestSelectArgs), _vp]
    L.la_quest_decode_fused.argtypes = [P(LaQuestDecodeArgs), _vp]
    L.la_topk_rows_workspace.argtypes = [P(LaTopkArgs)]
    L.la_topk_rows_workspace.restype = ctypes.c_size_t
    L.la_topk_rows.argtypes = [P(LaTopkArgs), _vp]
    L.la_indexer_topk_workspace.argtypes = [P(LaIndexerArgs)]
    L.la_indexer_topk_workspace.restype = ctypes.c_size_t
    L.la_indexer_topk.argtypes = [P(LaIndexerArgs), _vp]
    L.la_block_select_workspace.argtypes = [P(LaBlockSelectArgs)]
    L.la_block_select_workspace.restype = ctypes.c_size_t
    L.la_block_select.argtypes = [P(LaBlockSelectArgs), _vp]
    L.la_block_sparse_prefill_workspace.argtypes = [P(LaPrefillArgs)]
    L.la_block_sparse_prefill_workspace.restype = ctypes.c_size_t
    L.la_block_sparse_prefill.argtypes = [P(LaPrefillArgs), _vp]
    L.la_paged_kv_append.argtypes = [P(LaKvAppendArgs), _vp]
    L.la_gate_select_workspace.argtypes = [P(LaGateSelectArgs)]
    L.la_gate_select_workspace.restype = ctypes.c_size_t
    L.la_gate_select.argtypes = [P(LaGateSelectArgs), _vp]
    L.la_block_means.argtypes = [P(LaBlockMeansArgs), _vp]
    L.la_xattn_select_workspace.argtypes = [P(LaXattnSelectArgs)]
    L.la_xattn_select_workspace.restype = ctypes.c_size_t
    L.la_xattn_select.argtypes = [P(LaXattnSelectArgs), _vp]
    L.la_xattn_select.restype = ctypes.c_int
    L.la_device_status.argtypes = [ctypes.POINTER(ctypes.c_uint32), _i32, _vp]
    L.la_test_set_spin_limit.argtypes = [ctypes.c_uint32]
    for name in EXPORTED:
        fn = getattr(L, name)
        if fn.restype is None or fn.restype is ctypes.c_int:
            fn.restype = ctypes.c_int
    if L.la_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH}: ABI {L.la_abi_version()} != expected {ABI_VERSION}")
    _LIB = L
    return L


def check(rc: int, what: str) -> None:
    """Map a status code to the reference's exception types (ValueError for
    bad arguments, RuntimeError otherwise)."""
    if rc == LA_OK:
        return
    msg = (load().la_last_error() or b"").decode(errors="replace")
    if rc == LA_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: status {rc}: {msg}")


def device_status(device: Optional[torch.device] = None, clear: bool = True) -> int:
    """Status bits the kernels raised on ``device`` (LA_DEV_*), read after its
    current stream drains (a host synchronisation: for tests and debugging,
    not for hot loops)."""
    dev = device or torch.device("cuda", torch.cuda.current_device())
    bits = ctypes.c_uint32(0)
    with torch.cuda.device(dev):
        check(load().la_device_status(ctypes.byref(bits), 1 if clear else 0, stream_handle(dev)),
              "device_status")
    return int(bits.value)


_DT = {torch.float32: LA_F32, torch.bfloat16: LA_BF16, torch.float16: LA_F16,
       torch.float8_e4m3fn: LA_FP8_E4M3, torch.float64: LA_F64}


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DT[t]
    except KeyError:
        raise ValueError(f"unsupported dtype {t}") from None


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: Optional[torch.Tensor], what: str) -> torch.device:
    """Every tensor must live on the same GPU: there is no CPU fallback."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{what}: the HIP backend needs GPU tensors (got {t.device}); "
                               "the CPU oracle lives in oracle/ and is not a fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: tensors on {dev} and {t.device}")
    if dev is None:
        raise ValueError(f"{what}: no tensors")
    return dev


def workspace(nbytes: int, device: torch.device) -> Optional[torch.Tensor]:
    if nbytes <= 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)
