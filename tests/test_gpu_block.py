"""Block decode (kvl_mla_decode_compressed_block_bf16, src/mla_compressed_state.c:163-184, and
its Q8 counterpart): the tokens of a block run as one batch whose members share the state, and
the result must equal the serial single-token loop bit for bit -- the reference's exact
block-verify gate (src/exact_block_verify.c:359) -- at history lengths where the attention is
split over many workgroups."""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import Api, f32, rel_err, snapshot
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

L = lib.load()
O = Api(pyoracle.load_oracle(), "orc_")
KIMI = dict(inputs.KIMI)
TOL = 2e-3

KINDS = {
    "f32": (abi.KvlMlaCompressedState, "compressed_state", L.kvl_mla_decode_compressed_bf16,
            L.kvl_mla_decode_compressed_block_bf16, L.kvl_mla_compressed_state_fill_synthetic),
    "q8": (abi.KvlMlaCompressedQ8State, "compressed_q8_state", L.kvl_mla_decode_compressed_q8_bf16,
           L.kvl_mla_decode_compressed_q8_block_bf16, L.kvl_mla_compressed_q8_state_fill_synthetic),
}


def make_state(kind, cfg, cap, P, seed):
    cls, name, _, _, fill = KINDS[kind]
    st = cls()
    lib.check(getattr(L, f"kvl_mla_{name}_init")(C.byref(st), C.byref(cfg), cap), "init")
    lib.check(fill(C.byref(st), 0, P, seed), "fill")
    return st


# (kind, history rows, block tokens): the F32 case at 20000 rows needs more than 2048 splits for
# 9 lone plans, so the block runs as two groups
CASES = [("q8", 3000, 6), ("q8", 20000, 8), ("f32", 3000, 5), ("f32", 20000, 9)]


@pytest.mark.parametrize("kind,P,count", CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}" for c in CASES])
def test_block_equals_serial_long_history(kind, P, count):
    print(f"[block] {kind} history {P} block {count}", flush=True)
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xB1)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    x = np.ascontiguousarray(inputs.hidden(cfg, 0xB1 + P, count))
    _, name, single, block, _ = KINDS[kind]
    ser = make_state(kind, cfg, P + count, P, 0xB2)
    blk = make_state(kind, cfg, P + count, P, 0xB2)
    want = np.zeros((count, cfg.hidden_size), np.float32)
    for t in range(count):
        lib.check(single(f32(want[t]), f32(np.ascontiguousarray(x[t])), P + t, C.byref(cfg), C.byref(w),
                         C.byref(ser)), f"decode {t}")
    got = np.zeros_like(want)
    lib.check(block(f32(got), f32(x), count, P, C.byref(cfg), C.byref(w), C.byref(blk)), "block decode")
    assert ser.len == blk.len == P + count
    np.testing.assert_array_equal(got, want)
    a, b = snapshot(kind, blk, cfg), snapshot(kind, ser, cfg)
    for k in a:  # the appended rows (the history below P lives on the device only)
        np.testing.assert_array_equal(a[k][P:], b[k][P:], err_msg=k)
    assert rel_err(got, want) == 0.0
    # the oracle on the same history: its block decode for the FP32 state
    # (src/mla_compressed_state.c:163-184), its serial decodes for the Q8 state
    lib.check(getattr(L, f"kvl_mla_{name}_pull")(C.byref(blk), 0, P), "pull")
    ref_st = KINDS[kind][0]()
    assert getattr(O, f"mla_{name}_init")(C.byref(ref_st), C.byref(cfg), P + count) == 0
    fields = ({"codes": "latent_q8", "scale": "latent_scale", "rope": "rope_bf16"} if kind == "q8"
              else {"latent": "latent", "rope": "rope"})
    for k, v in snapshot(kind, blk, cfg).items():
        n = v[:P].size
        np.ctypeslib.as_array(getattr(ref_st, fields[k]), (n,))[:] = v[:P].ravel()
    ref_st.len = P
    ref = np.zeros_like(want)
    if kind == "f32":
        assert O.mla_decode_compressed_block_bf16(f32(ref), f32(x), count, P, C.byref(cfg), C.byref(w),
                                                  C.byref(ref_st)) == 0
    else:
        for t in range(count):
            assert O.mla_decode_compressed_q8_bf16(f32(ref[t]), f32(np.ascontiguousarray(x[t])), P + t, C.byref(cfg),
                                                   C.byref(w), C.byref(ref_st)) == 0
    e = rel_err(got, ref)
    print(f"[block]   vs oracle max|d|/max|ref| = {e:.3e}", flush=True)
    assert e <= TOL, e
    sa, so = snapshot(kind, blk, cfg), snapshot(kind, ref_st, cfg)
    if kind == "q8":  # appended rows: kv_a sums in another order, so codes may differ by one step
        dc = np.abs(sa["codes"][P:].astype(int) - so["codes"][P:].astype(int))
        assert dc.max() <= 1 and dc.mean() < 0.01, (dc.max(), dc.mean())
        np.testing.assert_allclose(sa["scale"][P:], so["scale"][P:], rtol=1e-5)
    else:
        for k in sa:
            assert rel_err(sa[k][P:], so[k][P:]) < 1e-4, k
    getattr(O, f"mla_{name}_free")(C.byref(ref_st))
    for st in (ser, blk):
        getattr(L, f"kvl_mla_{name}_free")(C.byref(st))
    L.kvl_mla_release_weights(C.byref(w))


def test_block_rejects_bad_arguments():
    """The reference's checks (src/mla_compressed_state.c:170-174): start must equal len and
    the block must fit; nothing is written."""
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xB3)
    w = layer.struct()
    st = make_state("q8", cfg, 10, 4, 0xB4)
    x = np.ascontiguousarray(inputs.hidden(cfg, 0xB3, 8))
    out = np.full((8, cfg.hidden_size), 3.0, np.float32)
    blk = L.kvl_mla_decode_compressed_q8_block_bf16
    assert blk(f32(out), f32(x), 2, 3, C.byref(cfg), C.byref(w), C.byref(st)) == -1   # start != len
    assert blk(f32(out), f32(x), 7, 4, C.byref(cfg), C.byref(w), C.byref(st)) == -1   # beyond capacity
    assert blk(f32(out), f32(x), 0, 4, C.byref(cfg), C.byref(w), C.byref(st)) == -1   # empty block
    assert st.len == 4 and np.all(out == 3.0)
    L.kvl_mla_compressed_q8_state_free(C.byref(st))
