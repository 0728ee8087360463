"""ctypes mirror of the kvl MLA C ABI (structs byte-identical to include/kvl/*.h).

The same prototypes describe three libraries that export the reference signatures:
the MI355X library (prefix ``kvl_``), the reference build used as a checker (``kvl_``) and the
CPU oracle (``orc_``). Struct layouts follow include/kvl/ops.h:17-34,
include/kvl/mla_state.h:13-22, include/kvl/mla_compressed_state.h:7-14 and
include/kvl/mla_compressed_q8_state.h:8-16 of the reference.
"""
import ctypes as C

c_int, c_float, c_size_t, c_void_p = C.c_int, C.c_float, C.c_size_t, C.c_void_p
f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)
i8p = C.POINTER(C.c_int8)


class KvlMlaConfig(C.Structure):
    _fields_ = [("hidden_size", c_int), ("num_heads", c_int), ("qk_nope_dim", c_int),
                ("qk_rope_dim", c_int), ("v_head_dim", c_int), ("kv_lora_rank", c_int),
                ("rms_eps", c_float), ("rope_theta", c_float)]


class KvlMlaBF16(C.Structure):
    _fields_ = [("q_proj", u16p), ("kv_a_proj", u16p), ("kv_a_norm", u16p),
                ("kv_b_proj", u16p), ("o_proj", u16p)]


class KvlMlaState(C.Structure):
    _fields_ = [("capacity", c_int), ("len", c_int), ("num_heads", c_int),
                ("qk_nope_dim", c_int), ("qk_rope_dim", c_int), ("v_head_dim", c_int),
                ("keys", f32p), ("values", f32p)]


class KvlMlaCompressedState(C.Structure):
    _fields_ = [("capacity", c_int), ("len", c_int), ("kv_lora_rank", c_int),
                ("qk_rope_dim", c_int), ("latent", f32p), ("rope", f32p)]


class KvlMlaCompressedQ8State(C.Structure):
    _fields_ = [("capacity", c_int), ("len", c_int), ("kv_lora_rank", c_int),
                ("qk_rope_dim", c_int), ("latent_q8", i8p), ("latent_scale", f32p),
                ("rope_bf16", u16p)]


class KvlMlaCompressedBF16State(C.Structure):
    """BF16-latent history of include/kvl/mla_hip.h (an extension: the FP32 state's layout with
    bf16 rows)."""
    _fields_ = [("capacity", c_int), ("len", c_int), ("kv_lora_rank", c_int),
                ("qk_rope_dim", c_int), ("latent", u16p), ("rope", u16p)]


CFG = C.POINTER(KvlMlaConfig)
W = C.POINTER(KvlMlaBF16)
ST = C.POINTER(KvlMlaState)
CS = C.POINTER(KvlMlaCompressedState)
QS = C.POINTER(KvlMlaCompressedQ8State)
BS = C.POINTER(KvlMlaCompressedBF16State)

# name (without prefix) -> (restype, argtypes)
REFERENCE_API = {
    "bf16_to_f32": (c_float, [C.c_uint16]),
    "matvec_bf16": (None, [f32p, f32p, u16p, c_int, c_int]),
    "rmsnorm_bf16": (None, [f32p, f32p, u16p, c_int, c_float]),
    "mla_state_init": (c_int, [ST, CFG, c_int]),
    "mla_state_reset": (None, [ST]),
    "mla_state_free": (None, [ST]),
    "mla_state_bytes": (c_size_t, [ST]),
    "mla_decode_bf16": (c_int, [f32p, f32p, c_int, CFG, W, ST]),
    "mla_compressed_state_init": (c_int, [CS, CFG, c_int]),
    "mla_compressed_state_reset": (None, [CS]),
    "mla_compressed_state_truncate": (c_int, [CS, c_int]),
    "mla_compressed_state_free": (None, [CS]),
    "mla_compressed_state_bytes": (c_size_t, [CS]),
    "mla_compressed_state_prefill_bf16": (c_int, [f32p, c_int, CFG, W, CS]),
    "mla_decode_compressed_bf16": (c_int, [f32p, f32p, c_int, CFG, W, CS]),
    "mla_decode_compressed_block_bf16": (c_int, [f32p, f32p, c_int, c_int, CFG, W, CS]),
    "mla_compressed_q8_state_init": (c_int, [QS, CFG, c_int]),
    "mla_compressed_q8_state_reset": (None, [QS]),
    "mla_compressed_q8_state_truncate": (c_int, [QS, c_int]),
    "mla_compressed_q8_state_free": (None, [QS]),
    "mla_compressed_q8_state_bytes": (c_size_t, [QS]),
    "mla_compressed_q8_state_prefill_bf16": (c_int, [f32p, c_int, CFG, W, QS]),
    "mla_decode_compressed_q8_bf16": (c_int, [f32p, f32p, c_int, CFG, W, QS]),
}
# the causal prefill entry point (include/kvl/ops.h:63-64)
PREFILL_API = {"mla_prefill_bf16": (c_int, [f32p, f32p, c_int, CFG, W])}


def declare(lib, table, prefix):
    """Attach restype/argtypes for every entry of ``table`` under ``prefix``."""
    for name, (res, args) in table.items():
        fn = getattr(lib, prefix + name)
        fn.restype = res
        fn.argtypes = args
    return lib


def ptr(arr, ctype):
    """Pointer to a C-contiguous numpy array's data."""
    assert arr.flags["C_CONTIGUOUS"]
    return arr.ctypes.data_as(C.POINTER(ctype))
