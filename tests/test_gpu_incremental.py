"""The reference's incremental gate on the GPU path (src/mla_incremental_probe.c:32-110): causal
prefill, expanded decode, compressed decode and "state prefill of 4 tokens, then decode token
5" give the same rows. The probe's own inputs (its sin/cos weight fill, :16-21, and hidden
states, :51-54) and its absolute gates (:103) are used on its shape; the Kimi-VL shapes, which
run the MFMA kernels, are held to the 2e-3 relative bar."""
import ctypes as C

import numpy as np
import pytest

from helpers import Api, decode_seq, f32, rel_err
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

L = lib.load()
G = Api(L, "kvl_")


def probe_bf16(n, scale, bias):
    """bf16 bits of bias + scale * (float)(sin(0.173 i) + 0.35 cos(0.071 i)), truncated (:10-21)."""
    i = np.arange(n, dtype=np.float64)
    v = (np.sin(i * 0.173) + 0.35 * np.cos(i * 0.071)).astype(np.float32)
    x = (np.float32(bias) + np.float32(scale) * v).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def probe_inputs():
    S, H, NH, DN, DR, DV, R = 5, 16, 2, 4, 4, 4, 6
    QO, KVO, KVB = NH * (DN + DR), R + DR, NH * (DN + DV)
    layer = inputs.Layer(q_proj=probe_bf16(QO * H, 0.037, 0.0), kv_a_proj=probe_bf16(KVO * H, 0.041, 0.0),
                         kv_a_norm=probe_bf16(R, 0.025, 0.93), kv_b_proj=probe_bf16(KVB * R, 0.052, 0.0),
                         o_proj=probe_bf16(H * NH * DV, 0.044, 0.0))
    t = np.arange(S, dtype=np.float64)[:, None]
    i = np.arange(H, dtype=np.float64)[None, :]
    x = (np.float32(0.17) * np.sin((t + 1) * (i + 2) * 0.11).astype(np.float32)
         + np.float32(0.03) * np.cos((i + 1) * 0.23).astype(np.float32)).astype(np.float32)
    cfg = abi.KvlMlaConfig(hidden_size=H, num_heads=NH, qk_nope_dim=DN, qk_rope_dim=DR, v_head_dim=DV,
                           kv_lora_rank=R, rms_eps=1e-6, rope_theta=10000.0)
    return cfg, layer, np.ascontiguousarray(x)


def test_probe_gate_expanded_compressed_batch_history():
    cfg, layer, x = probe_inputs()
    w = layer.struct()
    S, H, prefix = x.shape[0], x.shape[1], 4
    prefill = np.zeros((S, H), np.float32)
    assert G.prefill(prefill, x, S, cfg, w) == 0
    expanded, _ = decode_seq(G, "exp", cfg, w, x, capacity=S)
    compressed, _ = decode_seq(G, "f32", cfg, w, x, capacity=S)
    batch_next, _ = decode_seq(G, "f32", cfg, w, x, prefix=prefix, capacity=S)
    de = np.abs(prefill - expanded).max()
    dc = np.abs(prefill - compressed).max()
    db = np.abs(prefill[prefix] - batch_next[0]).max()
    print(f"[incremental] probe shape: expanded {de:.3e} compressed {dc:.3e} batch-history {db:.3e}"
          f" (max|out| {np.abs(prefill).max():.3e})", flush=True)
    assert de <= 1e-6 and dc <= 2e-6 and db <= 2e-6


def test_probe_gate_order_and_reset():
    """A decode at a position other than len fails; after reset, position 0 decodes again (:72-76)."""
    cfg, layer, x = probe_inputs()
    w = layer.struct()
    S, H = x.shape
    st = abi.KvlMlaState()
    assert G.mla_state_init(C.byref(st), C.byref(cfg), S) == 0
    out = np.zeros(H, np.float32)
    try:
        for t in range(S):
            assert G.mla_decode_bf16(f32(out), f32(np.ascontiguousarray(x[t])), t, C.byref(cfg), C.byref(w),
                                     C.byref(st)) == 0
        assert G.mla_decode_bf16(f32(out), f32(np.ascontiguousarray(x[0])), 0, C.byref(cfg), C.byref(w),
                                 C.byref(st)) == -1
        assert st.len == S
        G.mla_state_reset(C.byref(st))
        assert st.len == 0
        assert G.mla_decode_bf16(f32(out), f32(np.ascontiguousarray(x[0])), 0, C.byref(cfg), C.byref(w),
                                 C.byref(st)) == 0
        assert st.len == 1
    finally:
        G.mla_state_free(C.byref(st))


@pytest.mark.parametrize("kind", ["exp", "f32", "q8"])
def test_kimi_decode_rows_equal_prefill_rows(kind):
    """Kimi-VL shapes: every decode kind reproduces the causal prefill's rows (token t decoded
    over a history of t rows = prefill row t); the first half of the history comes from the
    state prefill for the compressed kinds."""
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.make_layer(cfg, 0xD1)
    w = layer.struct()
    S = 48
    x = inputs.hidden(cfg, 0xD1, S)
    prefill = np.zeros((S, cfg.hidden_size), np.float32)
    assert G.prefill(prefill, x, S, cfg, w) == 0
    prefix = 0 if kind == "exp" else S // 2
    dec, _ = decode_seq(G, kind, cfg, w, x, prefix=prefix)
    ref = prefill[prefix:].astype(np.float64)
    e = rel_err(dec, ref)
    rms = float(np.sqrt(np.sum((dec - ref) ** 2) / np.sum(ref ** 2)))
    print(f"[incremental] kimi {kind}: decode rows vs prefill rows max-rel {e:.3e} rel-rms {rms:.3e}",
          flush=True)
    assert np.all(np.isfinite(dec))
    if kind == "q8":
        # the int8 history against the fp32 prefill: the reference's own gate for this
        # comparison (src/spec_q8_lab_probe.c:131-132,177)
        assert rms <= 0.02 and np.abs(dec - ref).max() <= 0.02
    else:
        assert e <= 2e-3
