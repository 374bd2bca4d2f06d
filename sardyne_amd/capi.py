"""ctypes binding of libsardyne.so (the MI355X build).

``_SIGNATURES`` is the reference's binding table (sardyne/capi.py:33-102): the same 50 symbols with
the same argument and result types, so the reference's Python layer (runtime, CLI, server) binds
this library unchanged through ``SARDYNE_LIB``. ``_DEVICE_SIGNATURES`` adds the device-level entry
points of this build (weights and activations resident in GPU memory, HIP events) that tests and
the benchmark use; they have no counterpart in the reference.

The library is loaded on first use from ``SARDYNE_LIB`` or ``build/libsardyne.so``.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

_ROOT = pathlib.Path(__file__).resolve().parent.parent
_LIBNAME = "libsardyne.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u64 = ctypes.c_uint64
_lib = None


class _GGUFTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32), ("type", ctypes.c_uint32),
                ("ne", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]


class _GGUFKV(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("type", ctypes.c_uint32), ("arr_type", ctypes.c_uint32),
                ("n", ctypes.c_uint64), ("ptr", ctypes.c_void_p), ("str_pos", ctypes.c_void_p)]


class EngineModelInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in
                ("n_vocab", "dim", "n_layer", "n_head", "n_kv_head", "head_dim", "ffn_dim", "max_pos")] + \
               [("norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)] + \
               [(name, ctypes.c_int32) for name in ("rope_interleaved", "qkv_bias", "tied_embeddings", "qk_norm",
                                                     "n_expert", "n_expert_used", "ffn_exp_dim")]


_vp, _i32, _fp = ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_float)
_int, _sz = ctypes.c_int, ctypes.c_size_t

_SIGNATURES = {
    "engine_version": (ctypes.c_char_p, []),
    "engine_add_f32": (None, [_f32p, _f32p, _f32p, _sz]),
    "gguf_open": (_vp, [ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "gguf_close": (None, [_vp]),
    "gguf_version": (ctypes.c_uint32, [_vp]),
    "gguf_alignment": (ctypes.c_uint32, [_vp]),
    "gguf_data_offset": (_u64, [_vp]),
    "gguf_n_kv": (_u64, [_vp]),
    "gguf_n_tensors": (_u64, [_vp]),
    "gguf_get_kv": (ctypes.POINTER(_GGUFKV), [_vp, _u64]),
    "gguf_find_kv": (ctypes.c_int64, [_vp, ctypes.c_char_p]),
    "gguf_get_tensor": (ctypes.POINTER(_GGUFTensor), [_vp, _u64]),
    "gguf_find_tensor": (ctypes.c_int64, [_vp, ctypes.c_char_p]),
    "gguf_kv_get_u64": (_int, [_vp, ctypes.c_int64, ctypes.POINTER(_u64)]),
    "gguf_kv_get_f64": (_int, [_vp, ctypes.c_int64, ctypes.POINTER(ctypes.c_double)]),
    "gguf_kv_get_str": (_vp, [_vp, ctypes.c_int64, ctypes.POINTER(_u64)]),
    "gguf_kv_get_arr_str": (_vp, [_vp, ctypes.c_int64, _u64, ctypes.POINTER(_u64)]),
    "gguf_type_name": (ctypes.c_char_p, [ctypes.c_uint32]),
    "engine_model_load": (_vp, [ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "engine_model_free": (None, [_vp]),
    "engine_model_get_info": (None, [_vp, ctypes.POINTER(EngineModelInfo)]),
    "engine_ctx_new": (_vp, [_vp, _i32, _i32, _i32, _i32, ctypes.c_char_p, _sz]),
    "engine_ctx_n_threads": (_i32, [_vp]),
    "engine_ctx_free": (None, [_vp]),
    "engine_eval": (_int, [_vp, ctypes.POINTER(_i32), _i32]),
    "engine_logits": (_fp, [_vp]),
    "engine_n_logits": (_i32, [_vp]),
    "engine_n_past": (_i32, [_vp]),
    "engine_reset": (None, [_vp]),
    "engine_truncate": (_int, [_vp, _i32]),
    "engine_last_error": (ctypes.c_char_p, [_vp]),
    "op_simd": (_int, []),
    "op_set_simd": (_int, [_int]),
    "op_f16_to_f32_n": (None, [_vp, _vp, _sz]),
    "op_matmul_rows": (None, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int]),
    "op_dot_f32": (ctypes.c_float, [_vp, _vp, _int]),
    "op_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "op_row_to_f32": (None, [_vp, _int, _vp, _sz]),
    "op_row_size": (_sz, [_int, _int]),
    "op_quantize_rows": (None, [_int, _vp, _vp, _int, _int, _int]),
    "op_matmul_q_rows": (None, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int]),
    "op_vec_dot_q": (ctypes.c_float, [_int, _vp, _vp, _int]),
    "op_axpy": (None, [_vp, ctypes.c_float, _vp, _int]),
    "op_matmul": (None, [_vp, _vp, _vp, _int, _int, _int, _int]),
    "op_rmsnorm": (None, [_vp, _vp, _vp, _int, ctypes.c_float]),
    "op_softmax": (None, [_vp, _int]),
    "op_silu_mul": (None, [_vp, _vp, _int]),
    "op_rope_table": (None, [_vp, _vp, _int, _int, ctypes.c_float]),
    "op_rope": (None, [_vp, _int, _int, _vp, _vp, _int]),
    "op_attention": (None, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _vp]),
}


class SdyMat(ctypes.Structure):
    """Device-layout matrix descriptor (sdy_mat in sardyne_amd/csrc/sdy_shim.h)."""
    _fields_ = [("base", _vp), ("bytes", _sz), ("type", _int), ("n_in", _int), ("n_rows", ctypes.c_long),
                ("n_units", _int), ("plane_off", _sz * 5), ("gemm_ok", _int), ("gbase", _vp), ("gbytes", _sz),
                ("grow0", ctypes.c_long), ("grows", ctypes.c_long), ("hbase", _vp)]


class SdyBarrierStats(ctypes.Structure):
    """sdy_barrier_stats (include/sardyne.h)."""
    _fields_ = [("us_median", ctypes.c_float), ("us_mean", ctypes.c_float), ("us_mean_streaming", ctypes.c_float),
                ("kernel_ms", ctypes.c_float), ("rounds_done", _int), ("rounds_streaming", _int),
                ("timeouts", ctypes.c_uint), ("mismatches", ctypes.c_uint)]


class SdyMvArgs(ctypes.Structure):
    _fields_ = [("xq", _vp), ("x", _vp), ("n_tok", _int), ("out", _vp), ("out_stride", ctypes.c_long),
                ("bias", _vp), ("resid", _vp), ("row0", ctypes.c_long), ("row1", ctypes.c_long),
                ("epilogue", _int), ("nw", _vp), ("eps", ctypes.c_float), ("ws_ready", ctypes.c_int)]


_DEVICE_SIGNATURES = {
    "sdy_last_error": (ctypes.c_char_p, []),
    "op_last_error": (ctypes.c_char_p, []),
    "sdy_last_kernel": (ctypes.c_char_p, []),
    "sdy_init": (_int, []),
    "sdy_device_info": (_int, [ctypes.POINTER(_int), ctypes.POINTER(_sz)]),
    "sdy_grid_barrier_probe": (_int, [_int, _int, _int, _int, ctypes.POINTER(SdyBarrierStats)]),
    "sdy_kernel_boundary_us": (_int, [_int, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]),
    "sdy_mem_info": (_int, [ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "sdy_model_memory": (_int, [_vp, ctypes.POINTER(_sz), ctypes.POINTER(_sz), ctypes.POINTER(_int),
                                ctypes.POINTER(_int)]),
    "sdy_model_host_weights": (_int, [_vp, ctypes.POINTER(_sz), ctypes.POINTER(_int)]),
    "sdy_malloc": (_int, [ctypes.POINTER(_vp), _sz]),
    "sdy_free": (_int, [_vp]),
    "sdy_h2d": (_int, [_vp, _vp, _sz, _vp]),
    "sdy_d2h": (_int, [_vp, _vp, _sz, _vp]),
    "sdy_d2d": (_int, [_vp, _vp, _sz, _vp]),
    "sdy_memset": (_int, [_vp, _int, _sz, _vp]),
    "sdy_sync": (_int, [_vp]),
    "sdy_stream_new": (_int, [ctypes.POINTER(_vp)]),
    "sdy_stream_free": (_int, [_vp]),
    "sdy_event_new": (_int, [ctypes.POINTER(_vp)]),
    "sdy_event_record": (_int, [_vp, _vp]),
    "sdy_event_elapsed": (_int, [ctypes.POINTER(ctypes.c_float), _vp, _vp]),
    "sdy_event_free": (_int, [_vp]),
    "sdy_graph_begin": (_int, [_vp]),
    "sdy_graph_end": (_int, [_vp, ctypes.POINTER(_vp)]),
    "sdy_graph_launch": (_int, [_vp, _vp]),
    "sdy_graph_free": (_int, [_vp]),
    "sdy_membw_read": (_int, [_vp, _sz, _vp, _vp]),
    "sdy_membw_read_strided": (_int, [_vp, _sz, _vp, _vp]),
    "sdy_mat_bytes": (_sz, [_int, _int, ctypes.c_long]),
    "sdy_mat_upload": (_int, [ctypes.POINTER(SdyMat), _int, _int, ctypes.c_long, _vp, _vp]),
    "sdy_mat_upload_rows": (_int, [ctypes.POINTER(SdyMat), ctypes.c_long, ctypes.c_long, ctypes.c_long, _vp, _vp]),
    "sdy_mat_from_device": (_int, [ctypes.POINTER(SdyMat), _int, _int, ctypes.c_long, _vp, _vp]),
    "sdy_mat_free": (_int, [ctypes.POINTER(SdyMat)]),
    "sdy_mat_rows": (SdyMat, [ctypes.POINTER(SdyMat), ctypes.c_long, ctypes.c_long]),
    "sdy_dequant_rows": (_int, [ctypes.POINTER(SdyMat), ctypes.c_long, ctypes.c_long, _vp, _vp]),
    "sdy_quantize": (_int, [_int, _vp, _vp, _int, _int, _vp]),
    "sdy_matvec": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), _vp]),
    "sdy_mat_gemm_layout": (_int, [ctypes.POINTER(SdyMat), _vp]),
    "sdy_gemm2": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), ctypes.POINTER(SdyMat),
                         ctypes.POINTER(SdyMvArgs), _vp, _vp]),
    "sdy_matvec_pair_ok": (_int, [ctypes.POINTER(SdyMat), _int, ctypes.POINTER(SdyMat), _int]),
    "sdy_matvec_fused_ok": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), ctypes.POINTER(SdyMat),
                                   ctypes.POINTER(SdyMvArgs)]),
    "sdy_matvec_grouped_fused_ok": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), _int, ctypes.c_long,
                                           ctypes.c_long]),
    "sdy_matvec_pair": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), ctypes.POINTER(SdyMat),
                               ctypes.POINTER(SdyMvArgs), _vp]),
    "sdy_matvec_float": (_int, [_int, _vp, _int, ctypes.POINTER(SdyMvArgs), _vp]),
    "sdy_matvec_float_norm": (_int, [_int, _vp, _int, ctypes.POINTER(SdyMvArgs), _vp, _vp]),
    "sdy_matvec_grouped": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), _vp, _int, ctypes.c_long,
                                  ctypes.c_long, ctypes.c_long, _vp]),
    "sdy_matvec_grouped_route": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), _vp, _int, _int, _vp, _vp,
                                        ctypes.c_long, ctypes.c_long, ctypes.c_long, _vp]),
    "sdy_mat_alloc": (_int, [ctypes.POINTER(SdyMat), _int, _int, ctypes.c_long]),
    "sdy_mat_alloc_host": (_int, [ctypes.POINTER(SdyMat), _int, _int, ctypes.c_long]),
    "sdy_host_alloc_mapped": (_int, [ctypes.POINTER(_vp), ctypes.POINTER(_vp), _sz]),
    "sdy_host_free": (_int, [_vp]),
    "sdy_uploader_new": (_int, [ctypes.POINTER(_vp), _sz, _int, _int, _vp]),
    "sdy_uploader_rows": (_int, [_vp, ctypes.POINTER(SdyMat), ctypes.c_long, ctypes.c_long, ctypes.c_long,
                                 ctypes.c_long, ctypes.c_long, _vp]),
    "sdy_uploader_finish": (_int, [_vp]),
    "sdy_uploader_stats": (None, [_vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_double)]),
    "sdy_uploader_free": (_int, [_vp]),
    "sdy_mat_upload_map": (_int, [ctypes.POINTER(SdyMat), ctypes.c_long, ctypes.c_long, ctypes.c_long,
                                  ctypes.c_long, ctypes.c_long, _vp, _vp]),
    "sdy_rmsnorm": (_int, [_vp, _vp, _vp, _int, ctypes.c_float, _int, ctypes.c_long, ctypes.c_long, _vp]),
    "sdy_norm_quant": (_int, [_vp, _vp, ctypes.c_float, _int, _int, _vp, _int, _vp, _vp]),
    "sdy_attn_scores_floats": (_sz, [_int, _int, _int]),
    "sdy_kv_elt_bytes": (_sz, [_int]),
    "sdy_qk_rope_kv": (_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _int, _int, _int, _int, _int, _int,
                              _vp, _vp, _int, ctypes.c_long, _vp]),
    "sdy_qk_rope_kv_strided": (_int, [_vp, _vp, _vp, ctypes.c_long, ctypes.c_long, ctypes.c_long, _vp, _vp,
                                      ctypes.c_float, _vp, _vp, _int, _int, _int, _int, _int, _int, _vp, _vp, _int,
                                      ctypes.c_long, _vp]),
    "sdy_attention": (_int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int, ctypes.c_long, ctypes.c_long, _vp,
                             _vp, ctypes.c_long, _vp]),
    "sdy_attention_flash_ok": (_int, [_int, _int, _int]),
    "sdy_attention_flash": (_int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int, ctypes.c_long, ctypes.c_long,
                                   _vp, ctypes.c_long, _vp]),
    "sdy_quantize_gemm": (_int, [_vp, _vp, _int, _int, _vp, _vp]),
    "sdy_norm_quant_gemm": (_int, [_vp, _vp, ctypes.c_float, _int, _int, _vp, _vp, _vp, _vp]),
    "sdy_attn_decode_ok": (_int, [_int, _int, _int, _int]),
    "sdy_attn_decode_split_ok": (_int, [_int, _int, _int]),
    "sdy_attn_decode_split_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _int, _int, _int,
                                             _int, _vp, _vp, ctypes.c_long, _int, _vp, _vp, _vp]),
    "sdy_attn_decode_split_floats": (_sz, [_int, _int, _int]),
    "sdy_attn_decode_split": (_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _int, _int, _int, _int,
                                     _vp, _vp, ctypes.c_long, _int, _vp, _vp, _vp, _vp, _vp]),
    "sdy_attn_decode": (_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _int, _int, _int, _int, _vp,
                               _vp, _int, ctypes.c_long, _int, _vp, _vp, _vp, _vp]),
    "sdy_attn_chunked_ok": (_int, [_int, _int, _int]),
    "sdy_attn_chunked_floats": (_sz, [_int, _int, _int]),
    "sdy_attn_decode_chunked": (_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _int, _int, _int, _int,
                                       _vp, _vp, _int, ctypes.c_long, _int, _vp, _vp, _vp, _vp]),
    "sdy_moe_route": (_int, [_vp, _int, _int, _int, _vp, _vp, _vp]),
    "sdy_moe_combine": (_int, [_vp, _vp, _vp, _int, _int, _int, _vp, _vp, _vp]),
    "sdy_moe_down_combine": (_int, [ctypes.POINTER(SdyMat), _vp, _vp, _vp, _int, ctypes.c_long, _vp, _vp, _vp]),
    "sdy_gemm_ok": (_int, [ctypes.POINTER(SdyMat), _int]),
    "sdy_gemm_ws_bytes": (_sz, [_int, _int]),
    "sdy_gemm": (_int, [ctypes.POINTER(SdyMat), ctypes.POINTER(SdyMvArgs), _vp, _vp]),
    "sdy_gemm_grouped_tile": (_int, []),
    "sdy_gemm_grouped": (_int, [ctypes.POINTER(SdyMat), ctypes.c_long, _int, _vp, _vp, _vp, _vp, _int,
                                ctypes.POINTER(SdyMvArgs), _vp, _vp]),
    "sdy_moe_sort": (_int, [_vp, _int, _int, _int, _int, _vp, _vp, _vp, _vp, _vp]),
    "sdy_gather_rows": (_int, [_vp, _vp, _int, _int, _vp, _vp]),
}

EPI_NONE, EPI_SWIGLU = 0, 1
KV_F32, KV_F16 = 0, 1


def lib_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get("SARDYNE_LIB", _ROOT / "build" / _LIBNAME))


def available() -> bool:
    return lib_path().exists()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = lib_path()
        if not path.exists():
            raise OSError(f"{path} non trovata: compilare la libreria con `make` (python -m sardyne_amd.build)")
        handle = ctypes.CDLL(str(path))
        for table in (_SIGNATURES, _DEVICE_SIGNATURES):
            for name, (res, args) in table.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def version() -> str:
    return lib().engine_version().decode()


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    assert a.shape == b.shape
    out = np.empty_like(a)
    lib().engine_add_f32(a, b, out, a.size)
    return out


# ---------------------------------------------------------------- device-level helpers (tests, bench)

class GPUError(RuntimeError):
    pass


def check(rc: int):
    if rc != 0:
        raise GPUError(lib().sdy_last_error().decode(errors="replace"))


class DeviceBuffer:
    """A device allocation owned by Python (freed on close/garbage collection)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _vp()
        check(lib().sdy_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(lib().sdy_h2d(b.ptr, a.ctypes.data, a.nbytes, stream))
        check(lib().sdy_sync(stream))
        return b

    def to_array(self, dtype, shape, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype)
        check(lib().sdy_d2h(out.ctypes.data, self.ptr, out.nbytes, stream))
        check(lib().sdy_sync(stream))
        return out

    def close(self):
        if self.ptr:
            lib().sdy_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceMatrix:
    """A quantized (or float) weight matrix in the device layout."""

    def __init__(self, type_id: int, n_in: int, n_rows: int, raw: np.ndarray, stream=None, gemm_layout=True):
        self.m = SdyMat()
        raw = np.ascontiguousarray(raw).view(np.uint8)
        check(lib().sdy_mat_upload(ctypes.byref(self.m), type_id, n_in, n_rows, raw.ctypes.data, stream))
        if gemm_layout:  # the prefill GEMM's copy (Q4_K / Q6_K), as the engine makes it after loading
            check(lib().sdy_mat_gemm_layout(ctypes.byref(self.m), stream))
        self.type, self.n_in, self.n_rows = type_id, n_in, n_rows

    def close(self):
        if self.m.base:
            lib().sdy_mat_free(ctypes.byref(self.m))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
