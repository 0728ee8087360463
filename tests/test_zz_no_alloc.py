"""kvl_mla_decode_compressed_q8_batch_device_noalloc against the allocating entry point it
mirrors (kvl_mla_decode_compressed_q8_batch_device): the same outputs and appended rows, bit
for bit, on two calls in a row (the second with fewer, shorter sequences, so stale contents of
the shared device scratch would show), plus its refusals. Runs alone in a fresh process too:
it warms up through the allocating call first, as a no-allocation caller does."""
import ctypes as C

import numpy as np
import pytest

from helpers import snapshot
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

L = lib.load()
Q8P = C.POINTER(abi.KvlMlaCompressedQ8State)


def make_states(cfg, lens, seed):
    sts = []
    for i, n in enumerate(lens):
        st = abi.KvlMlaCompressedQ8State()
        assert L.kvl_mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), int(n) + 2) == 0
        lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, int(n), seed + i), "fill")
        sts.append(st)
    return sts


def run(fn, cfg, w, states, x, flags):
    B = len(states)
    arr = (Q8P * B)(*[C.pointer(s) for s in states])
    d_x = L.kvl_mla_device_alloc(x.nbytes)
    d_o = L.kvl_mla_device_alloc(x.nbytes)
    assert d_x and d_o
    lib.check(L.kvl_mla_copy_to_device(d_x, x.ctypes.data, x.nbytes), "h2d")
    junk = np.full_like(x, 5.0)
    lib.check(L.kvl_mla_copy_to_device(d_o, junk.ctypes.data, x.nbytes), "h2d")
    rc = fn(d_o, d_x, B, C.byref(cfg), C.byref(w), arr, flags)
    lib.check(rc, fn.__name__)
    out = np.zeros_like(x)
    lib.check(L.kvl_mla_copy_to_host(out.ctypes.data, d_o, x.nbytes), "d2h")
    for st in states:
        lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, st.len), "pull")
    L.kvl_mla_device_free(d_x)
    L.kvl_mla_device_free(d_o)
    return out


def test_noalloc_decode_equals_allocating_decode():
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.make_layer(cfg, 0xA7)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    # call 1: 12 ragged sequences (splits from several workgroups each); call 2: 3 shorter ones
    for call, lens in enumerate(([9000, 31000, 700, 5000, 17000, 64, 2500, 12000, 30000, 1, 4096, 800],
                                 [300, 2000, 65])):
        print(f"[noalloc] call {call}: {len(lens)} sequences, {sum(lens)} rows", flush=True)
        x = np.ascontiguousarray(inputs.hidden(cfg, 0xA8 + call, len(lens), tag="q"))
        ref_states = make_states(cfg, lens, 0xA00 + 100 * call)
        new_states = make_states(cfg, lens, 0xA00 + 100 * call)
        ref = run(L.kvl_mla_decode_compressed_q8_batch_device, cfg, w, ref_states, x, 0)
        got = run(L.kvl_mla_decode_compressed_q8_batch_device_noalloc, cfg, w, new_states, x, 0)
        np.testing.assert_array_equal(got, ref, err_msg=f"call {call}")
        for a, b in zip(new_states, ref_states):
            assert a.len == b.len
            sa, sb = snapshot("q8", a, cfg), snapshot("q8", b, cfg)
            for k in sa:
                np.testing.assert_array_equal(sa[k], sb[k], err_msg=f"call {call} {k}")
        # residual form: out += attention(x), in place
        h = run(L.kvl_mla_decode_compressed_q8_batch_device, cfg, w, ref_states, x, lib.RESIDUAL | lib.NO_ADVANCE)
        g = run(L.kvl_mla_decode_compressed_q8_batch_device_noalloc, cfg, w, new_states, x,
                lib.RESIDUAL | lib.NO_ADVANCE)
        np.testing.assert_array_equal(g, h, err_msg=f"call {call} residual")
        for st in ref_states + new_states:
            L.kvl_mla_compressed_q8_state_free(C.byref(st))
    L.kvl_mla_release_weights(C.byref(w))


def test_noalloc_refusals():
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.make_layer(cfg, 0xA9)
    w = layer.struct()
    x = np.ascontiguousarray(inputs.hidden(cfg, 0xA9, 17, tag="q"))
    states = make_states(cfg, [100] * 17, 0xB00)
    d_x = L.kvl_mla_device_alloc(x.nbytes)
    nx = L.kvl_mla_decode_compressed_q8_batch_device_noalloc
    arr = (Q8P * 17)(*[C.pointer(s) for s in states])
    assert nx(d_x, d_x, 1, C.byref(cfg), C.byref(w), arr, 0) == -1       # weights not bound
    assert "bound" in lib.last_error()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    assert nx(d_x, d_x, 17, C.byref(cfg), C.byref(w), arr, 0) == -1      # batch beyond 16
    assert "16" in lib.last_error()
    fresh = abi.KvlMlaCompressedQ8State()
    assert L.kvl_mla_compressed_q8_state_init(C.byref(fresh), C.byref(cfg), 8) == 0
    one = (Q8P * 1)(C.pointer(fresh))
    assert nx(d_x, d_x, 1, C.byref(cfg), C.byref(w), one, 0) == -1       # no device copy yet
    assert fresh.len == 0 and all(s.len == 100 for s in states)
    L.kvl_mla_compressed_q8_state_free(C.byref(fresh))
    L.kvl_mla_device_free(d_x)
    for st in states:
        L.kvl_mla_compressed_q8_state_free(C.byref(st))
    L.kvl_mla_release_weights(C.byref(w))
