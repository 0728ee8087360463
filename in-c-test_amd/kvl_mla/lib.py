"""Loader of libkvl_mla.so, the MI355X MLA library (C ABI of include/kvl/*.h).

The library is built in-tree by ``__graft_entry__.build()`` (in-c-test_amd/csrc/Makefile).
There is no fallback: a missing library raises, so nothing silently runs elsewhere.
"""
import ctypes as C
import os

from . import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkvl_mla.so")

QSP = C.POINTER(abi.QS)
CSP = C.POINTER(abi.CS)
BSP = C.POINTER(abi.BS)

# include/kvl/mla_hip.h
EXT_API = {
    "mla_last_error": (C.c_char_p, []),
    "mla_init": (C.c_int, []),
    "mla_bind_weights": (C.c_int, [abi.CFG, abi.W]),
    "mla_release_weights": (C.c_int, [abi.W]),
    "mla_compressed_state_sync": (C.c_int, [abi.CS]),
    "mla_compressed_q8_state_sync": (C.c_int, [abi.QS]),
    "mla_state_sync": (C.c_int, [abi.ST]),
    "mla_decode_compressed_batch_bf16": (C.c_int, [abi.f32p, abi.f32p, C.POINTER(C.c_int), C.c_int,
                                                   abi.CFG, abi.W, CSP]),
    "mla_decode_compressed_q8_batch_bf16": (C.c_int, [abi.f32p, abi.f32p, C.POINTER(C.c_int),
                                                      C.c_int, abi.CFG, abi.W, QSP]),
    "mla_decode_compressed_q8_block_bf16": (C.c_int, [abi.f32p, abi.f32p, C.c_int, C.c_int, abi.CFG, abi.W,
                                                      abi.QS]),
    "mla_decode_compressed_q8_batch_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG,
                                                        abi.W, QSP, C.c_uint]),
    "mla_decode_compressed_batch_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG,
                                                     abi.W, CSP, C.c_uint]),
    "mla_decode_compressed_q8_batch_device_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG,
                                                                abi.W, QSP, C.c_uint]),
    "mla_attention_layer_q8_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W, abi.u16p,
                                                 abi.u16p, QSP, C.c_uint]),
    "mla_attention_layer_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W, abi.u16p,
                                              abi.u16p, CSP, C.c_uint]),
    "mla_prefill_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W]),
    "mla_prefill_range_status": (C.c_int, []),
    "mla_prefill_compressed_state_bf16": (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W, abi.CS]),
    "mla_prefill_compressed_q8_state_bf16": (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W, abi.QS]),
    "mla_prefill_compressed_state_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W,
                                                      abi.CS]),
    "mla_prefill_compressed_q8_state_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W,
                                                         abi.QS]),
    "mla_stream": (C.c_void_p, []),
    "mla_synchronize": (C.c_int, []),
    "mla_device_alloc": (C.c_void_p, [C.c_size_t]),
    "mla_device_free": (C.c_int, [C.c_void_p]),
    "mla_copy_to_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "mla_copy_to_host": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "mla_capture_begin": (C.c_int, []),
    "mla_capture_end": (C.c_int, [C.POINTER(C.c_void_p)]),
    "mla_graph_launch": (C.c_int, [C.c_void_p]),
    "mla_graph_destroy": (C.c_int, [C.c_void_p]),
    "mla_timing_enable": (C.c_int, [C.c_int]),
    "mla_set_fused_qprep": (C.c_int, [C.c_int]),
    "mla_set_fused_combine": (C.c_int, [C.c_int]),
    "mla_set_fused_projection": (C.c_int, [C.c_int]),
    "mla_set_fused_wait_limit": (C.c_int, [C.c_uint]),
    "mla_timing_stages": (C.c_int, [C.c_uint]),
    "mla_timing_read": (C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_int)]),
    "mla_event_record": (C.c_void_p, []),
    "mla_event_elapsed_ms": (C.c_double, [C.c_void_p, C.c_void_p]),
    "mla_event_destroy": (C.c_int, [C.c_void_p]),
    "mla_copy_kernel": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "mla_read_kernel": (C.c_int, [C.c_void_p, C.c_size_t]),
    "mla_empty_kernel": (C.c_int, []),
    "mla_q8_pack_rows": (C.c_int, [abi.i8p, abi.f32p, abi.u16p, abi.f32p, abi.f32p,
                                   C.POINTER(C.c_int), C.c_int, C.c_int, C.c_int, C.c_float]),
    "mla_compressed_q8_state_fill_synthetic": (C.c_int, [abi.QS, C.c_int, C.c_int, C.c_uint64]),
    "mla_compressed_state_fill_synthetic": (C.c_int, [abi.CS, C.c_int, C.c_int, C.c_uint64]),
    "mla_compressed_q8_state_pull": (C.c_int, [abi.QS, C.c_int, C.c_int]),
    "mla_compressed_state_pull": (C.c_int, [abi.CS, C.c_int, C.c_int]),
    # BF16-latent state
    "mla_compressed_bf16_state_init": (C.c_int, [abi.BS, abi.CFG, C.c_int]),
    "mla_compressed_bf16_state_reset": (None, [abi.BS]),
    "mla_compressed_bf16_state_truncate": (C.c_int, [abi.BS, C.c_int]),
    "mla_compressed_bf16_state_free": (None, [abi.BS]),
    "mla_compressed_bf16_state_bytes": (C.c_size_t, [abi.BS]),
    "mla_compressed_bf16_state_sync": (C.c_int, [abi.BS]),
    "mla_compressed_bf16_state_prefill_bf16": (C.c_int, [abi.f32p, C.c_int, abi.CFG, abi.W, abi.BS]),
    "mla_decode_compressed_bf16_bf16": (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W, abi.BS]),
    "mla_decode_compressed_bf16_block_bf16": (C.c_int, [abi.f32p, abi.f32p, C.c_int, C.c_int, abi.CFG, abi.W,
                                                        abi.BS]),
    "mla_decode_compressed_bf16_batch_bf16": (C.c_int, [abi.f32p, abi.f32p, C.POINTER(C.c_int), C.c_int,
                                                        abi.CFG, abi.W, BSP]),
    "mla_decode_compressed_bf16_batch_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W,
                                                          BSP, C.c_uint]),
    "mla_compressed_bf16_state_fill_synthetic": (C.c_int, [abi.BS, C.c_int, C.c_int, C.c_uint64]),
    "mla_compressed_bf16_state_pull": (C.c_int, [abi.BS, C.c_int, C.c_int]),
    "mla_prefill_compressed_bf16_state_bf16": (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W, abi.BS]),
    "mla_prefill_compressed_bf16_state_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W,
                                                           abi.BS]),
    "mla_attention_layer_bf16_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, abi.CFG, abi.W, abi.u16p,
                                                   abi.u16p, BSP, C.c_uint]),
}

# stage 1 is the fused append + query preparation of the compressed formats (the expanded
# format times them as stages 1 and 2)
STAGES = ("gemv_in", "append_qprep", "qprep", "attention", "combine", "gemv_out")
RESIDUAL = 1
NO_ADVANCE = 2

_lib = None


def load():
    """libkvl_mla with every prototype declared; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python __graft_entry__.py` (build)")
        lib = C.CDLL(LIB_PATH)
        abi.declare(lib, abi.REFERENCE_API, "kvl_")
        abi.declare(lib, abi.PREFILL_API, "kvl_")
        abi.declare(lib, EXT_API, "kvl_")
        _lib = lib
    return _lib


def last_error():
    e = load().kvl_mla_last_error()
    return e.decode() if e else ""


def check(rc, what="call"):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {last_error()}")
