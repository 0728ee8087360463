"""Drivers that run the same call sequence against any library exporting the reference API
(the MI355X library, the reference build, or the oracle with prefix ``orc_``)."""
import ctypes as C

import numpy as np

from kvl_mla import abi
from kvl_mla.inputs import bf16_bits_to_f32


class Api:
    """Uniform access to ``<prefix>name`` functions of a loaded library."""

    def __init__(self, lib, prefix):
        self.lib, self.prefix = lib, prefix

    def __getattr__(self, name):
        return getattr(self.lib, self.prefix + name)

    def prefill(self, out, x, S, cfg, w):
        fn = getattr(self.lib, self.prefix + "mla_prefill_bf16", None)
        if fn is None:
            fn = self.lib.orc_mla_prefill_streaming
        return fn(f32(out), f32(x), S, C.byref(cfg), C.byref(w))


def f32(a):
    return abi.ptr(a, C.c_float)


def u16(a):
    return abi.ptr(a, C.c_uint16)


def i8(a):
    return abi.ptr(a, C.c_int8)


def decode_seq(api, kind, cfg, w, x, start=0, prefix=0, capacity=None):
    """Run ``prefix`` tokens through the state prefill-fill (if >0), then decode the remaining
    tokens of x one by one. Returns (outputs [n, H], state snapshot dict)."""
    S, H = x.shape
    cap = capacity or S + 1
    st = {"exp": abi.KvlMlaState, "f32": abi.KvlMlaCompressedState,
          "q8": abi.KvlMlaCompressedQ8State}[kind]()
    init = {"exp": api.mla_state_init, "f32": api.mla_compressed_state_init,
            "q8": api.mla_compressed_q8_state_init}[kind]
    dec = {"exp": api.mla_decode_bf16, "f32": api.mla_decode_compressed_bf16,
           "q8": api.mla_decode_compressed_q8_bf16}[kind]
    assert init(C.byref(st), C.byref(cfg), cap) == 0
    if prefix:
        fill = {"f32": api.mla_compressed_state_prefill_bf16,
                "q8": api.mla_compressed_q8_state_prefill_bf16}[kind]
        assert fill(f32(x[:prefix]), prefix, C.byref(cfg), C.byref(w), C.byref(st)) == 0
    outs = np.zeros((S - prefix, H), dtype=np.float32)
    for t in range(prefix, S):
        rc = dec(f32(outs[t - prefix]), f32(np.ascontiguousarray(x[t])), t, C.byref(cfg),
                 C.byref(w), C.byref(st))
        assert rc == 0, f"decode failed at t={t}"
    snap = snapshot(kind, st, cfg)
    free = {"exp": api.mla_state_free, "f32": api.mla_compressed_state_free,
            "q8": api.mla_compressed_q8_state_free}[kind]
    free(C.byref(st))
    return outs, snap


def snapshot(kind, st, cfg):
    L = st.len
    R, DR = cfg.kv_lora_rank, cfg.qk_rope_dim
    if kind == "f32":
        return {"latent": np.ctypeslib.as_array(st.latent, (L * R,)).copy().reshape(L, R),
                "rope": np.ctypeslib.as_array(st.rope, (L * DR,)).copy().reshape(L, DR)}
    if kind == "q8":
        return {"codes": np.ctypeslib.as_array(st.latent_q8, (L * R,)).copy().reshape(L, R),
                "scale": np.ctypeslib.as_array(st.latent_scale, (L,)).copy(),
                "rope": np.ctypeslib.as_array(st.rope_bf16, (L * DR,)).copy().reshape(L, DR)}
    NH, QD, DV = cfg.num_heads, cfg.qk_nope_dim + cfg.qk_rope_dim, cfg.v_head_dim
    return {"keys": np.ctypeslib.as_array(st.keys, (L * NH * QD,)).copy(),
            "values": np.ctypeslib.as_array(st.values, (L * NH * DV,)).copy()}


def rel_err(got, ref):
    """max|got-ref| / max|ref| -- the attention-output parity metric."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def dequant(snap):
    return snap["codes"].astype(np.float32) * snap["scale"][:, None]


def rope_f32(snap):
    return bf16_bits_to_f32(snap["rope"])
