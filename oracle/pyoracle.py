"""Loader of the CPU checkers -- TEST INFRASTRUCTURE ONLY.

Used by tests/, the smoke check and the CPU-baseline leg of bench.py. Two checkers exist:

* the oracle restatement (``build/liborc.so``, functions ``orc_*``), always built;
* the reference MLA path compiled from its own sources (``_ref/libkvl_ref_{avx2,scalar}.so``,
  functions ``kvl_*``), present when the sources were available at build time.
"""
import ctypes as C
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(ROOT, "in-c-test_amd"))

from kvl_mla import abi  # noqa: E402

ORACLE_SO = os.path.join(HERE, "build", "liborc.so")
REF_SO = {"avx2": os.path.join(HERE, "_ref", "libkvl_ref_avx2.so"),
          "scalar": os.path.join(HERE, "_ref", "libkvl_ref_scalar.so")}
ORDER = {"scalar": 0, "avx2": 1}

_EXTRA = {
    "set_order": (None, [C.c_int]),
    "get_order": (C.c_int, []),
    "f32_to_bf16_rne": (C.c_uint16, [C.c_float]),
    "rope_interleaved": (None, [abi.f32p, abi.f32p, C.c_int, C.c_int, C.c_float]),
    "quantize_latent": (None, [abi.i8p, abi.f32p, abi.f32p, C.c_int]),
    "dequant": (C.c_float, [C.c_int8, C.c_float]),
    "q8_pack_row": (None, [abi.i8p, abi.f32p, abi.u16p, abi.f32p, abi.f32p, C.c_int, C.c_int,
                           C.c_int, C.c_float]),
    "q8_row_from_katmp": (None, [abi.i8p, abi.f32p, abi.u16p, abi.f32p, abi.u16p, C.c_int,
                                 C.c_int, C.c_float, C.c_int, C.c_float]),
    "mla_prefill_streaming": (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W]),
    "mla_prefill_materialized": (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W]),
    "mla_prefill_streaming_rows": (C.c_int, [abi.f32p, abi.f32p, C.c_int, C.POINTER(C.c_int), C.c_int,
                                             abi.CFG, abi.W]),
    "mla_decode_compressed_bf16_rows": (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W, abi.CS]),
}

_cache = {}


def load_oracle():
    """The oracle restatement; raises if it has not been built (oracle/Makefile)."""
    if "orc" not in _cache:
        if not os.path.exists(ORACLE_SO):
            raise FileNotFoundError(f"{ORACLE_SO} missing: run `make -C oracle oracle`")
        lib = C.CDLL(ORACLE_SO)
        abi.declare(lib, abi.REFERENCE_API, "orc_")
        abi.declare(lib, _EXTRA, "orc_")
        _cache["orc"] = lib
    return _cache["orc"]


def load_reference(kind="avx2"):
    """The reference build of the given kind, or None when it was not built."""
    key = "ref_" + kind
    if key not in _cache:
        path = REF_SO[kind]
        if not os.path.exists(path):
            _cache[key] = None
        else:
            lib = C.CDLL(path)
            abi.declare(lib, abi.REFERENCE_API, "kvl_")
            abi.declare(lib, abi.PREFILL_API, "kvl_")
            abi.declare(lib, {"mla_prefill_materialized_bf16":
                              (C.c_int, [abi.f32p, abi.f32p, C.c_int, abi.CFG, abi.W])}, "kvl_")
            _cache[key] = lib
    return _cache[key]
