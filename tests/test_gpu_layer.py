"""The attention half of a decoder layer on the device (kvl_mla_attention_layer[_q8]_device):
n1 = RMSNorm(h, input_norm); h += attention(n1); n2 = RMSNorm(h, post_attn_norm), as
src/generate.c:34-67 (attention_token) computes it per token.

Bars: bit-identical to the same composition through this library's host API (kvl_rmsnorm_bf16,
the batched decode, an fp32 add); against the oracle's composition, the attention increment and
n2 within max|d|/max|ref| <= 2e-3."""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import f32, rel_err, u16
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

TOL = 2e-3
ORC = pyoracle.load_oracle()
L = lib.load()
KIMI = dict(inputs.KIMI)

KINDS = {
    "f32": (abi.KvlMlaCompressedState, "mla_compressed_state", "mla_decode_compressed_bf16",
            "mla_decode_compressed_batch_bf16", "mla_attention_layer_device"),
    "q8": (abi.KvlMlaCompressedQ8State, "mla_compressed_q8_state", "mla_decode_compressed_q8_bf16",
           "mla_decode_compressed_q8_batch_bf16", "mla_attention_layer_q8_device"),
}


def prefilled(api, prefix, kind, cfg, w, prompts, cap):
    cls, name, _, _, _ = KINDS[kind]
    out = []
    for p in prompts:
        st = cls()
        assert getattr(api, prefix + name + "_init")(C.byref(st), C.byref(cfg), cap) == 0
        assert getattr(api, prefix + name + "_prefill_bf16")(f32(p), p.shape[0], C.byref(cfg), C.byref(w),
                                                             C.byref(st)) == 0
        out.append(st)
    return out


@pytest.mark.parametrize("kind", ["f32", "q8"])
def test_attention_layer_matches_host_composition_and_oracle(kind):
    print(f"[layer] {kind}", flush=True)
    cfg = inputs.config(**KIMI)
    H = cfg.hidden_size
    layer = inputs.make_layer(cfg, 0xA1)
    w = layer.struct()
    rng = np.random.default_rng(0xA1)
    in_norm = inputs.f32_to_bf16_bits(1.0 + 0.02 * rng.standard_normal(H).astype(np.float32))
    post_norm = inputs.f32_to_bf16_bits(1.0 + 0.02 * rng.standard_normal(H).astype(np.float32))
    lens = [40, 57, 64]
    B = len(lens)
    prompts = [np.ascontiguousarray(inputs.hidden(cfg, 0xA2 + i, n) * np.float32(0.3)) for i, n in enumerate(lens)]
    h0 = np.ascontiguousarray(inputs.hidden(cfg, 0xA3, B))
    cap = max(lens) + 2
    cls, name, single, batch, fused = KINDS[kind]
    P = C.POINTER(cls)

    # device layer
    dev_states = prefilled(L, "kvl_", kind, cfg, w, prompts, cap)
    arr = (P * B)(*[C.pointer(s) for s in dev_states])
    nb = h0.nbytes
    d_h, d_n2 = L.kvl_mla_device_alloc(nb), L.kvl_mla_device_alloc(nb)
    assert d_h and d_n2
    lib.check(L.kvl_mla_copy_to_device(d_h, h0.ctypes.data, nb), "h2d")
    lib.check(getattr(L, "kvl_" + fused)(d_h, d_n2, B, C.byref(cfg), C.byref(w), u16(in_norm), u16(post_norm),
                                         arr, 0), "attention layer")
    h1 = np.zeros_like(h0)
    n2 = np.zeros_like(h0)
    lib.check(L.kvl_mla_copy_to_host(h1.ctypes.data, d_h, nb), "d2h")
    lib.check(L.kvl_mla_copy_to_host(n2.ctypes.data, d_n2, nb), "d2h")
    assert [s.len for s in dev_states] == [n + 1 for n in lens]

    # the same composition through the host API
    host_states = prefilled(L, "kvl_", kind, cfg, w, prompts, cap)
    harr = (P * B)(*[C.pointer(s) for s in host_states])
    n1 = np.zeros_like(h0)
    for b in range(B):
        L.kvl_rmsnorm_bf16(f32(n1[b]), f32(h0[b]), u16(in_norm), H, np.float32(cfg.rms_eps))
    attn = np.zeros_like(h0)
    pos = np.array(lens, np.int32)
    lib.check(getattr(L, "kvl_" + batch)(f32(attn), f32(n1), pos.ctypes.data_as(C.POINTER(C.c_int)), B,
                                         C.byref(cfg), C.byref(w), harr), "host batch decode")
    r1 = (h0 + attn).astype(np.float32)
    n2h = np.zeros_like(h0)
    for b in range(B):
        L.kvl_rmsnorm_bf16(f32(n2h[b]), f32(r1[b]), u16(post_norm), H, np.float32(cfg.rms_eps))
    np.testing.assert_array_equal(h1, r1)
    np.testing.assert_array_equal(n2, n2h)

    # the oracle's composition (src/generate.c:52-64 restated)
    orc_states = prefilled(ORC, "orc_", kind, cfg, w, prompts, cap)
    attn_o = np.zeros_like(h0)
    n2o = np.zeros_like(h0)
    for b in range(B):
        n1o = np.zeros(H, np.float32)
        ORC.orc_rmsnorm_bf16(f32(n1o), f32(h0[b]), u16(in_norm), H, C.c_float(cfg.rms_eps))
        assert getattr(ORC, "orc_" + single)(f32(attn_o[b]), f32(n1o), lens[b], C.byref(cfg), C.byref(w),
                                             C.byref(orc_states[b])) == 0
        r1o = (h0[b] + attn_o[b]).astype(np.float32)
        ORC.orc_rmsnorm_bf16(f32(n2o[b]), f32(r1o), u16(post_norm), H, C.c_float(cfg.rms_eps))
    e_attn, e_n2 = rel_err(h1 - h0, attn_o), rel_err(n2, n2o)
    print(f"[layer]   attention increment {e_attn:.3e}, n2 {e_n2:.3e}", flush=True)
    assert e_attn <= TOL and e_n2 <= TOL

    L.kvl_mla_device_free(d_h)
    L.kvl_mla_device_free(d_n2)
    for sts, api, pre in ((dev_states, L, "kvl_"), (host_states, L, "kvl_"), (orc_states, ORC, "orc_")):
        for s in sts:
            getattr(api, pre + name + "_free")(C.byref(s))


def test_attention_layer_rejects_bad_arguments():
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xA4)
    w = layer.struct()
    norm = inputs.f32_to_bf16_bits(np.ones(cfg.hidden_size, np.float32))
    st = abi.KvlMlaCompressedQ8State()
    assert L.kvl_mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), 4) == 0
    arr = (C.POINTER(abi.KvlMlaCompressedQ8State) * 1)(C.pointer(st))
    d, e = L.kvl_mla_device_alloc(cfg.hidden_size * 4), L.kvl_mla_device_alloc(cfg.hidden_size * 4)
    fn = L.kvl_mla_attention_layer_q8_device
    assert fn(d, d, 1, C.byref(cfg), C.byref(w), u16(norm), u16(norm), arr, 0) == -1      # n2 aliases h
    assert fn(d, e, 1, C.byref(cfg), C.byref(w), u16(norm), u16(norm), arr, lib.RESIDUAL) == -1  # flag
    assert fn(d, e, 0, C.byref(cfg), C.byref(w), u16(norm), u16(norm), arr, 0) == -1      # empty batch
    assert st.len == 0
    L.kvl_mla_device_free(d)
    L.kvl_mla_device_free(e)
    L.kvl_mla_compressed_q8_state_free(C.byref(st))
