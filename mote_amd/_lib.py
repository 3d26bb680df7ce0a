"""ctypes binding of libmote_relation.so (include/mote_relation.h).

The structures below mirror the header field by field. `lib()` loads the in-tree library once and
raises if it is missing: there is no fallback path. Calls pass raw device pointers and the current
HIP stream of the tensors' device.
"""

from __future__ import annotations

import ctypes as C
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libmote_relation.so")

MOTE_OK = 0
MOTE_F32 = 0
MOTE_BF16 = 1
MOTE_DECODE_ADVANCE = 1
MOTE_DECODE_ROPE_F32 = 2
MOTE_DECODE_STATIC_BYTES = 1 << 20
MOTE_DECODE_STATIC_SLOTS = 4
MOTE_BWD_ROWS, MOTE_BWD_KEYS, MOTE_BWD_FINISH, MOTE_BWD_QUERIES = 1, 2, 4, 8

_DTYPES = {torch.float32: MOTE_F32, torch.bfloat16: MOTE_BF16}


class View(C.Structure):
    _fields_ = [("data", C.c_void_p), ("stride_b", C.c_int64), ("stride_h", C.c_int64), ("stride_r", C.c_int64)]


class FwdArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("H", C.c_int), ("TQ", C.c_int), ("TK", C.c_int), ("D", C.c_int),
        ("q_start", C.c_int), ("tau_s", C.c_float),
        ("p1", View), ("p2", View), ("info", View), ("y", View),
        ("ibar", C.c_void_p), ("lse", C.c_void_p), ("g", C.c_void_p), ("lam", C.c_void_p),
        ("cu_seqlens", C.c_void_p), ("total_rows", C.c_int),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class BwdArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("H", C.c_int), ("TQ", C.c_int), ("TK", C.c_int), ("D", C.c_int),
        ("q_start", C.c_int), ("tau_s", C.c_float), ("deterministic", C.c_int),
        ("p1", View), ("p2", View), ("info", View), ("dy", View),
        ("ibar", C.c_void_p), ("lse", C.c_void_p), ("g", C.c_void_p),
        ("dp1", View), ("dp2", View), ("dinfo", View),
        ("dlam", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("stages", C.c_int),
    ]


class RopeArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("T", C.c_int), ("H", C.c_int), ("D", C.c_int), ("pos0", C.c_int),
        ("layer_parity", C.c_int), ("inv_freq", C.c_void_p), ("theta", C.c_void_p),
        ("qkv", C.c_void_p), ("qkv_sb", C.c_int64), ("qkv_sr", C.c_int64),
        ("p1", View), ("p2", View), ("info", View),
    ]


class RopeBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("T", C.c_int), ("H", C.c_int), ("D", C.c_int), ("pos0", C.c_int),
        ("layer_parity", C.c_int), ("inv_freq", C.c_void_p), ("theta", C.c_void_p),
        ("qkv", C.c_void_p), ("qkv_sb", C.c_int64), ("qkv_sr", C.c_int64), ("qkv_info_only", C.c_int),
        ("dp1", View), ("dp2", View), ("dinfo", View),
        ("dqkv", C.c_void_p), ("dqkv_sb", C.c_int64), ("dqkv_sr", C.c_int64),
        ("dtheta", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class DecodeArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("H", C.c_int), ("D", C.c_int), ("capacity", C.c_int),
        ("layer_parity", C.c_int), ("flags", C.c_int), ("tau_s", C.c_float),
        ("lam", C.c_void_p), ("inv_freq", C.c_void_p), ("theta", C.c_void_p), ("S", C.c_void_p),
        ("p1", C.c_void_p), ("p2", C.c_void_p), ("info", C.c_void_p), ("in_sb", C.c_int64),
        ("cache_p2", View), ("cache_info", View),
        ("y", C.c_void_p), ("y_sb", C.c_int64), ("g", C.c_void_p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t), ("xm", C.c_void_p), ("run", C.c_void_p),
        ("static_slot", C.c_int),
    ]


class NormArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("res_dtype", C.c_int), ("out_dtype", C.c_int), ("res_out_dtype", C.c_int),
        ("rows", C.c_int), ("D", C.c_int), ("eps", C.c_float),
        ("x", C.c_void_p), ("x_sr", C.c_int64), ("residual", C.c_void_p), ("res_sr", C.c_int64),
        ("weight", C.c_void_p), ("y", C.c_void_p), ("y_sr", C.c_int64),
        ("residual_out", C.c_void_p), ("res_out_sr", C.c_int64), ("rstd", C.c_void_p),
    ]


class NormBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("dres_out_dtype", C.c_int), ("s_dtype", C.c_int), ("dx_dtype", C.c_int),
        ("dres_dtype", C.c_int), ("rows", C.c_int), ("D", C.c_int),
        ("dy", C.c_void_p), ("dy_sr", C.c_int64), ("dres_out", C.c_void_p), ("dres_out_sr", C.c_int64),
        ("s", C.c_void_p), ("s_sr", C.c_int64), ("rstd", C.c_void_p), ("weight", C.c_void_p),
        ("dx", C.c_void_p), ("dx_sr", C.c_int64), ("dresidual", C.c_void_p), ("dres_sr", C.c_int64),
        ("dweight", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class QkvRopeArgs(C.Structure):
    _fields_ = [
        ("B", C.c_int), ("T", C.c_int), ("H", C.c_int), ("D", C.c_int), ("pos0", C.c_int), ("layer_parity", C.c_int),
        ("x", C.c_void_p), ("x_sb", C.c_int64), ("x_sr", C.c_int64), ("w", C.c_void_p), ("w_sr", C.c_int64),
        ("inv_freq", C.c_void_p), ("theta", C.c_void_p), ("p1", View), ("p2", View), ("info", View),
        ("info_raw", C.c_void_p), ("ir_sb", C.c_int64), ("ir_sr", C.c_int64),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t), ("table_ready", C.c_int),
        ("norm_w1", C.c_void_p), ("norm_w2", C.c_void_p), ("norm_eps", C.c_float),
        ("qk_raw", C.c_void_p), ("qr_sb", C.c_int64), ("qr_sr", C.c_int64),
    ]


class HeadNormBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("rows", C.c_int), ("parts", C.c_int), ("H", C.c_int), ("D", C.c_int), ("eps", C.c_float),
        ("x", C.c_void_p), ("x_sr", C.c_int64), ("dy", C.c_void_p), ("dy_sr", C.c_int64),
        ("dx", C.c_void_p), ("dx_sr", C.c_int64), ("gain0", C.c_void_p), ("gain1", C.c_void_p),
        ("dgain0", C.c_void_p), ("dgain1", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class GateProductArgs(C.Structure):
    _fields_ = [
        ("B", C.c_int), ("T", C.c_int), ("D", C.c_int), ("x", C.c_void_p), ("x_sr", C.c_int64),
        ("w", C.c_void_p), ("w_sr", C.c_int64), ("y", C.c_void_p), ("y_sr", C.c_int64),
        ("z", C.c_void_p), ("s", C.c_void_p), ("z_sr", C.c_int64),
    ]


class SkinnyGemmArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("N", C.c_int), ("K", C.c_int),
        ("x", C.c_void_p), ("x_sr", C.c_int64), ("w", C.c_void_p), ("w_sr", C.c_int64),
        ("y", C.c_void_p), ("y_sr", C.c_int64), ("run", C.c_void_p),
        ("g", C.c_void_p), ("xm", C.c_void_p), ("heads", C.c_int),
    ]


class WgradArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("M", C.c_int), ("N", C.c_int), ("K", C.c_int),
        ("a", C.c_void_p), ("a_sr", C.c_int64), ("x", C.c_void_p), ("x_sr", C.c_int64),
        ("dw", C.c_void_p), ("dw_sr", C.c_int64), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class PageCopyArgs(C.Structure):
    _fields_ = [
        ("to_page", C.c_int), ("planes", C.c_int), ("H", C.c_int), ("D", C.c_int), ("elem_bytes", C.c_int),
        ("rows", C.c_int), ("arena", C.c_void_p), ("a_plane", C.c_int64), ("a_head", C.c_int64),
        ("arena_row0", C.c_int), ("page", C.c_void_p), ("p_plane", C.c_int64), ("p_head", C.c_int64),
        ("page_row0", C.c_int),
    ]


class ChunkRouteArgs(C.Structure):
    _fields_ = [
        ("B", C.c_int), ("L", C.c_int), ("mask", C.c_void_p), ("mask_sr", C.c_int64),
        ("cum", C.c_void_p), ("perm", C.c_void_p), ("num", C.c_void_p), ("cu_seqlens", C.c_void_p),
    ]


class ChunkGatherArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("L", C.c_int), ("M", C.c_int), ("D", C.c_int),
        ("hidden", C.c_void_p), ("h_sb", C.c_int64), ("h_sr", C.c_int64),
        ("perm", C.c_void_p), ("num", C.c_void_p), ("cu_seqlens", C.c_void_p),
        ("out", C.c_void_p), ("o_sb", C.c_int64), ("o_sr", C.c_int64),
    ]


class ChunkGatherBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("B", C.c_int), ("L", C.c_int), ("M", C.c_int), ("D", C.c_int),
        ("dout", C.c_void_p), ("g_sb", C.c_int64), ("g_sr", C.c_int64),
        ("mask", C.c_void_p), ("mask_sr", C.c_int64), ("cum", C.c_void_p), ("num", C.c_void_p),
        ("cu_seqlens", C.c_void_p), ("dhidden", C.c_void_p), ("dh_sb", C.c_int64), ("dh_sr", C.c_int64),
    ]


class DechunkArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("prob_dtype", C.c_int), ("out_dtype", C.c_int),
        ("B", C.c_int), ("L", C.c_int), ("M", C.c_int), ("D", C.c_int), ("eps", C.c_float),
        ("hidden", C.c_void_p), ("h_sb", C.c_int64), ("h_sr", C.c_int64),
        ("prob", C.c_void_p), ("p_sb", C.c_int64), ("p_sr", C.c_int64),
        ("perm", C.c_void_p), ("num", C.c_void_p), ("cum", C.c_void_p), ("init", C.c_void_p),
        ("out", C.c_void_p), ("o_sb", C.c_int64), ("o_sr", C.c_int64), ("w", C.c_void_p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class DechunkBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("prob_dtype", C.c_int), ("dout_dtype", C.c_int), ("dx_dtype", C.c_int),
        ("dprob_dtype", C.c_int), ("B", C.c_int), ("L", C.c_int), ("M", C.c_int), ("D", C.c_int),
        ("eps", C.c_float),
        ("dout", C.c_void_p), ("g_sb", C.c_int64), ("g_sr", C.c_int64),
        ("hidden", C.c_void_p), ("h_sb", C.c_int64), ("h_sr", C.c_int64),
        ("prob", C.c_void_p), ("p_sb", C.c_int64), ("p_sr", C.c_int64),
        ("perm", C.c_void_p), ("num", C.c_void_p), ("mask", C.c_void_p), ("mask_sr", C.c_int64),
        ("cum", C.c_void_p), ("w", C.c_void_p),
        ("dhidden", C.c_void_p), ("dh_sb", C.c_int64), ("dh_sr", C.c_int64),
        ("dprob", C.c_void_p), ("dp_sb", C.c_int64), ("dp_sr", C.c_int64),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class DechunkStepArgs(C.Structure):
    _fields_ = [
        ("prob_dtype", C.c_int), ("hidden_dtype", C.c_int), ("state_dtype", C.c_int),
        ("B", C.c_int), ("D", C.c_int), ("eps", C.c_float),
        ("mask", C.c_void_p), ("prob", C.c_void_p), ("p_sr", C.c_int64),
        ("hidden", C.c_void_p), ("h_sr", C.c_int64), ("last_value", C.c_void_p), ("l_sr", C.c_int64),
        ("out", C.c_void_p), ("o_sr", C.c_int64),
    ]


# every symbol the header declares, with its argument types
EXPORTS = {
    "mote_last_error": ([], C.c_char_p),
    "mote_version": ([], C.c_char_p),
    "mote_relation_fwd_workspace": ([C.POINTER(FwdArgs)], C.c_size_t),
    "mote_relation_fwd": ([C.POINTER(FwdArgs), C.c_void_p], C.c_int),
    "mote_relation_bwd_workspace": ([C.POINTER(BwdArgs)], C.c_size_t),
    "mote_relation_bwd": ([C.POINTER(BwdArgs), C.c_void_p], C.c_int),
    "mote_rope_givens_fwd": ([C.POINTER(RopeArgs), C.c_void_p], C.c_int),
    "mote_rope_givens_bwd_workspace": ([C.POINTER(RopeBwdArgs)], C.c_size_t),
    "mote_rope_givens_bwd": ([C.POINTER(RopeBwdArgs), C.c_void_p], C.c_int),
    "mote_relation_decode_workspace": ([C.POINTER(DecodeArgs)], C.c_size_t),
    "mote_relation_decode": ([C.POINTER(DecodeArgs), C.c_void_p], C.c_int),
    "mote_relation_decode_static": ([C.POINTER(DecodeArgs), C.c_void_p], C.c_int),
    "mote_add_rms_norm_fwd": ([C.POINTER(NormArgs), C.c_void_p], C.c_int),
    "mote_add_rms_norm_bwd_workspace": ([C.POINTER(NormBwdArgs)], C.c_size_t),
    "mote_add_rms_norm_bwd": ([C.POINTER(NormBwdArgs), C.c_void_p], C.c_int),
    "mote_qkv_rope_workspace": ([C.POINTER(QkvRopeArgs)], C.c_size_t),
    "mote_qkv_rope_fwd": ([C.POINTER(QkvRopeArgs), C.c_void_p], C.c_int),
    "mote_gate_product": ([C.POINTER(GateProductArgs), C.c_void_p], C.c_int),
    "mote_head_rms_norm_bwd_workspace": ([C.POINTER(HeadNormBwdArgs)], C.c_size_t),
    "mote_head_rms_norm_bwd": ([C.POINTER(HeadNormBwdArgs), C.c_void_p], C.c_int),
    "mote_skinny_gemm": ([C.POINTER(SkinnyGemmArgs), C.c_void_p], C.c_int),
    "mote_wgrad_workspace": ([C.POINTER(WgradArgs)], C.c_size_t),
    "mote_wgrad": ([C.POINTER(WgradArgs), C.c_void_p], C.c_int),
    "mote_arena_page_copy": ([C.POINTER(PageCopyArgs), C.c_void_p], C.c_int),
    "mote_chunk_route": ([C.POINTER(ChunkRouteArgs), C.c_void_p], C.c_int),
    "mote_chunk_gather": ([C.POINTER(ChunkGatherArgs), C.c_void_p], C.c_int),
    "mote_chunk_gather_bwd": ([C.POINTER(ChunkGatherBwdArgs), C.c_void_p], C.c_int),
    "mote_dechunk_workspace": ([C.POINTER(DechunkArgs)], C.c_size_t),
    "mote_dechunk_fwd": ([C.POINTER(DechunkArgs), C.c_void_p], C.c_int),
    "mote_dechunk_bwd_workspace": ([C.POINTER(DechunkBwdArgs)], C.c_size_t),
    "mote_dechunk_bwd": ([C.POINTER(DechunkBwdArgs), C.c_void_p], C.c_int),
    "mote_dechunk_step": ([C.POINTER(DechunkStepArgs), C.c_void_p], C.c_int),
    "mote_abi_layout": ([], C.c_char_p),
    "mote_clock_probe": ([C.c_void_p, C.c_int, C.c_int, C.c_void_p], C.c_int),
}

# the header's struct behind each ctypes mirror (checked against mote_abi_layout() by the tests)
STRUCTS = {
    "mote_view": View, "mote_relation_fwd_args": FwdArgs, "mote_relation_bwd_args": BwdArgs,
    "mote_rope_givens_args": RopeArgs, "mote_rope_givens_bwd_args": RopeBwdArgs,
    "mote_relation_decode_args": DecodeArgs, "mote_add_rms_norm_args": NormArgs,
    "mote_add_rms_norm_bwd_args": NormBwdArgs, "mote_qkv_rope_args": QkvRopeArgs,
    "mote_gate_product_args": GateProductArgs, "mote_head_norm_bwd_args": HeadNormBwdArgs, "mote_skinny_gemm_args": SkinnyGemmArgs,
    "mote_wgrad_args": WgradArgs,
    "mote_page_copy_args": PageCopyArgs, "mote_chunk_route_args": ChunkRouteArgs,
    "mote_chunk_gather_args": ChunkGatherArgs, "mote_chunk_gather_bwd_args": ChunkGatherBwdArgs,
    "mote_dechunk_args": DechunkArgs, "mote_dechunk_bwd_args": DechunkBwdArgs,
    "mote_dechunk_step_args": DechunkStepArgs,
}


def abi_layout() -> dict:
    """{struct: (size, {field: (offset, size)})} as the library's compiler laid the header out."""
    out = {}
    for line in lib().mote_abi_layout().decode().splitlines():
        head, *fields = line.split(";")
        name, size = head.split()
        out[name] = (int(size), {f.split()[0]: (int(f.split()[1]), int(f.split()[2])) for f in fields})
    return out

_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"libmote_relation.so is not built ({LIB_PATH}); run `python -m mote_amd.build` "
                        "(the Relation path has no fallback without it)")
                handle = C.CDLL(LIB_PATH)
                for name, (argtypes, restype) in EXPORTS.items():
                    fn = getattr(handle, name)
                    fn.argtypes = argtypes
                    fn.restype = restype
                _lib = handle
    return _lib


def available() -> bool:
    return os.path.exists(LIB_PATH)


def check(rc: int, what: str) -> None:
    if rc != MOTE_OK:
        msg = lib().mote_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"Relation kernels take float32 or bfloat16 tensors, got {t.dtype}") from None


def view(t: torch.Tensor) -> View:
    """A [B, H, rows, D] tensor as a mote_view (unit stride along D required)."""
    assert t.dim() == 4 and t.stride(3) == 1, "last axis must be contiguous"
    return View(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
