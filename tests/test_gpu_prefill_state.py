"""Prefill with the state fill of the same tokens (kvl_mla_prefill_compressed[_q8]_state_*),
the call sequence of src/generate.c:208-210 (kvl_mla_prefill_bf16, then the state prefill of
src/mla_compressed_state.c:52-84 / src/mla_compressed_q8_state.c:129-159) as one call.

Bars: output and state rows bit-identical to the two separate calls of this library; against
the oracle, outputs max|got - ref| / max|ref| <= 2e-3 and state rows within the rounding of
the kv_a projection (the Q8 codes of a row move by at most one step)."""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import Api, decode_seq, f32, rel_err, snapshot
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

TOL = 2e-3
ORC = pyoracle.load_oracle()
O = Api(ORC, "orc_")
L = lib.load()
G = Api(L, "kvl_")

STREAM = dict(hidden_size=16, num_heads=2, qk_nope_dim=4, qk_rope_dim=4, v_head_dim=8,
              kv_lora_rank=6, rms_eps=1e-5, rope_theta=800000.0)  # src/mla_streaming_probe.c:39,46
KIMI = dict(inputs.KIMI)

STATE = {"f32": (abi.KvlMlaCompressedState, "mla_compressed_state"),
         "q8": (abi.KvlMlaCompressedQ8State, "mla_compressed_q8_state")}
FUSED = {"f32": "mla_prefill_compressed_state", "q8": "mla_prefill_compressed_q8_state"}


def new_state(api, kind, cfg, cap):
    cls, name = STATE[kind]
    st = cls()
    assert getattr(api, name + "_init")(C.byref(st), C.byref(cfg), cap) == 0
    return st


def free_state(api, kind, st):
    getattr(api, STATE[kind][1] + "_free")(C.byref(st))


def separate(kind, cfg, w, x, cap):
    S, H = x.shape
    out = np.zeros((S, H), np.float32)
    lib.check(L.kvl_mla_prefill_bf16(f32(out), f32(x), S, C.byref(cfg), C.byref(w)), "prefill")
    st = new_state(G, kind, cfg, cap)
    lib.check(getattr(G, STATE[kind][1] + "_prefill_bf16")(f32(x), S, C.byref(cfg), C.byref(w), C.byref(st)),
              "state prefill")
    return out, st


def fused(kind, cfg, w, x, cap):
    S, H = x.shape
    out = np.zeros((S, H), np.float32)
    st = new_state(G, kind, cfg, cap)
    lib.check(getattr(G, FUSED[kind] + "_bf16")(f32(out), f32(x), S, C.byref(cfg), C.byref(w), C.byref(st)),
              "fused prefill")
    return out, st


def assert_snap_equal(a, b):
    assert a.keys() == b.keys()
    for k in a:
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)


CASES = [("stream", STREAM, 37, 0.2, False), ("kimi", KIMI, 130, 0.02, False), ("kimi", KIMI, 300, 0.02, True)]


@pytest.mark.parametrize("name,dims,S,std,bf16_x", CASES, ids=[f"{c[0]}-{c[2]}" for c in CASES])
@pytest.mark.parametrize("kind", ["f32", "q8"])
def test_fused_equals_prefill_then_state_prefill(name, dims, S, std, bf16_x, kind):
    """State bit-identical to the state prefill's. Generic route (stream-probe shapes, the fill
    computes its own kv_a): output bit-identical too. Kimi-VL MFMA route (one kv_a for the
    attention and the state, in the decode's summation order): output within 5e-4 of the plain
    prefill's (a last-bit change of kv_a can move the bf8 rounding of a score correction
    operand, 2^-14 of |K||Q|; each output is within 2e-3 of the oracle's). S not a multiple of
    the tiles."""
    print(f"[fused] {kind} {name} S={S}", flush=True)
    cfg = inputs.config(**dims)
    layer = inputs.make_layer(cfg, 0xF0 + S, std=std)
    w = layer.struct()
    x = inputs.hidden(cfg, 0xF0 + S, S, bf16_exact=bf16_x)
    oa, sa = separate(kind, cfg, w, x, S + 3)
    ob, sb = fused(kind, cfg, w, x, S + 3)
    assert sa.len == sb.len == S
    if name == "stream":
        np.testing.assert_array_equal(ob, oa)
    else:
        print(f"[fused]   vs plain prefill max|d|/max|ref| = {rel_err(ob, oa):.3e}", flush=True)
        assert rel_err(ob, oa) <= 5e-4
    assert_snap_equal(snapshot(kind, sb, cfg), snapshot(kind, sa, cfg))
    free_state(G, kind, sa)
    free_state(G, kind, sb)


@pytest.mark.parametrize("kind", ["f32", "q8"])
def test_fused_then_decode_matches_oracle(kind):
    """Prompt of 200 tokens through the fused call, then 3 decode tokens, against the oracle's
    prefill, state prefill and decode."""
    print(f"[fused] {kind} prompt 200 + decode 3 vs oracle", flush=True)
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xF7)
    w = layer.struct()
    P, T = 200, 3
    x = inputs.hidden(cfg, 0xF7, P + T)
    xp = np.ascontiguousarray(x[:P])
    out, st = fused(kind, cfg, w, xp, P + T + 1)
    ref = np.zeros_like(out)
    assert ORC.orc_mla_prefill_streaming(f32(ref), f32(xp), P, C.byref(cfg), C.byref(w)) == 0
    assert rel_err(out, ref) <= TOL, rel_err(out, ref)
    # state rows against the oracle's state prefill of the same tokens
    ost = new_state(O, kind, cfg, P + T + 1)
    assert getattr(O, STATE[kind][1] + "_prefill_bf16")(f32(xp), P, C.byref(cfg), C.byref(w), C.byref(ost)) == 0
    got, exp = snapshot(kind, st, cfg), snapshot(kind, ost, cfg)
    if kind == "f32":
        assert rel_err(got["latent"], exp["latent"]) <= 1e-5
    else:
        dc = np.abs(got["codes"].astype(np.int32) - exp["codes"].astype(np.int32))
        assert dc.max() <= 1 and np.mean(dc) <= 1e-2, (dc.max(), np.mean(dc))
        np.testing.assert_allclose(got["scale"], exp["scale"], rtol=1e-5)
    if kind == "q8":  # BF16 keys: one rounding step of 2^-8 at most
        assert rel_err(inputs.bf16_bits_to_f32(got["rope"]), inputs.bf16_bits_to_f32(exp["rope"])) <= 1e-2
    else:
        assert rel_err(got["rope"], exp["rope"]) <= 1e-5
    free_state(O, kind, ost)
    # decode continues from the fused state; the oracle from its own
    dec = getattr(G, "mla_decode_compressed_bf16" if kind == "f32" else "mla_decode_compressed_q8_bf16")
    outs = np.zeros((T, cfg.hidden_size), np.float32)
    for t in range(T):
        assert dec(f32(outs[t]), f32(np.ascontiguousarray(x[P + t])), P + t, C.byref(cfg), C.byref(w),
                   C.byref(st)) == 0
    refs, _ = decode_seq(O, kind, cfg, w, x, prefix=P)
    print(f"[fused]   decode max|d|/max|ref| = {rel_err(outs, refs):.3e}", flush=True)
    assert rel_err(outs, refs) <= TOL
    # and equals this library's own separate calls followed by the same decode
    mine, _ = decode_seq(G, kind, cfg, w, x, prefix=P)
    np.testing.assert_array_equal(outs, mine)
    free_state(G, kind, st)


@pytest.mark.parametrize("kind", ["f32", "q8"])
def test_fused_device_variant_matches_host_variant(kind):
    print(f"[fused] {kind} device variant S=257", flush=True)
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xF9)
    w = layer.struct()
    S = 257
    x = np.ascontiguousarray(inputs.hidden(cfg, 0xF9, S))
    oh, sh = fused(kind, cfg, w, x, S)
    sd = new_state(G, kind, cfg, S)
    nbytes = x.nbytes
    dx, dout = L.kvl_mla_device_alloc(nbytes), L.kvl_mla_device_alloc(nbytes)
    assert dx and dout
    lib.check(L.kvl_mla_copy_to_device(dx, x.ctypes.data, nbytes), "h2d")
    lib.check(getattr(G, FUSED[kind] + "_device")(dout, dx, S, C.byref(cfg), C.byref(w), C.byref(sd)),
              "fused device")
    od = np.zeros_like(x)
    lib.check(L.kvl_mla_copy_to_host(od.ctypes.data, dout, nbytes), "d2h")
    assert sd.len == S
    pull = L.kvl_mla_compressed_state_pull if kind == "f32" else L.kvl_mla_compressed_q8_state_pull
    lib.check(pull(C.byref(sd), 0, S), "pull")
    np.testing.assert_array_equal(od, oh)
    assert_snap_equal(snapshot(kind, sd, cfg), snapshot(kind, sh, cfg))
    L.kvl_mla_device_free(dx)
    L.kvl_mla_device_free(dout)
    free_state(G, kind, sh)
    free_state(G, kind, sd)


def test_fused_rejects_bad_arguments():
    """The state prefill's checks (empty state, seq_len within capacity); nothing written."""
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xFA)
    w = layer.struct()
    x = inputs.hidden(cfg, 0xFA, 8)
    out = np.full((8, cfg.hidden_size), 7.0, np.float32)
    st = new_state(G, "q8", cfg, 4)
    assert L.kvl_mla_prefill_compressed_q8_state_bf16(f32(out), f32(x), 8, C.byref(cfg), C.byref(w), C.byref(st)) == -1
    assert st.len == 0 and np.all(out == 7.0)
    lib.check(L.kvl_mla_prefill_compressed_q8_state_bf16(f32(out), f32(x), 2, C.byref(cfg), C.byref(w),
                                                         C.byref(st)), "fused")
    assert st.len == 2
    assert L.kvl_mla_prefill_compressed_q8_state_bf16(f32(out), f32(x), 2, C.byref(cfg), C.byref(w), C.byref(st)) == -1
    assert st.len == 2
    free_state(G, "q8", st)
