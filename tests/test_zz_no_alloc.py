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
    for st in states:
        L.kvl_mla_compressed_q8_state_free(C.byref(st))
    # a split plan whose partials overflow the fixed array: 16 sequences of 50,000 rows make
    # 16 x 48 splits of 32.9 KB (25 MB > 24 MiB). The RoPE table is built first by an allocating
    # call, so the partials are what is refused.
    print("[noalloc] refusals: partials beyond the fixed array, position beyond the RoPE table", flush=True)
    big = make_states(cfg, [50000] * 16, 0xB40)
    barr = (Q8P * 16)(*[C.pointer(s) for s in big])
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xB4, 16, tag="q"))
    d_b = L.kvl_mla_device_alloc(xb.nbytes)
    lib.check(L.kvl_mla_copy_to_device(d_b, xb.ctypes.data, xb.nbytes), "h2d")
    lib.check(L.kvl_mla_decode_compressed_q8_batch_device(d_b, d_b, 1, C.byref(cfg), C.byref(w), barr,
                                                          lib.NO_ADVANCE), "allocating call")
    assert nx(d_b, d_b, 16, C.byref(cfg), C.byref(w), barr, 0) == -1
    assert "partials" in lib.last_error(), lib.last_error()
    assert all(s.len == 50000 for s in big)
    for st in big:
        L.kvl_mla_compressed_q8_state_free(C.byref(st))
    # a position no allocating call has reached: the RoPE table (grown by those calls in powers
    # of two, 65,536 positions at most in these tests) does not cover it
    far = make_states(cfg, [150000], 0xB50)
    farr = (Q8P * 1)(C.pointer(far[0]))
    assert nx(d_b, d_b, 1, C.byref(cfg), C.byref(w), farr, 0) == -1
    assert "RoPE table" in lib.last_error(), lib.last_error()
    assert far[0].len == 150000
    L.kvl_mla_compressed_q8_state_free(C.byref(far[0]))
    L.kvl_mla_device_free(d_b)
    L.kvl_mla_device_free(d_x)
    L.kvl_mla_release_weights(C.byref(w))


def test_noalloc_under_capture_and_after_a_larger_plan():
    """The entry point under graph capture on the library stream (capture refuses every device
    allocation the library would make, so a stray one fails the capture), its replays against
    the eager call, and a call whose split plan is larger than the allocating calls before it
    made: it must not move library memory, so a graph captured before it still launches."""
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.make_layer(cfg, 0xAB)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    small = make_states(cfg, [3000, 1200], 0xC00)
    sarr = (Q8P * 2)(*[C.pointer(s) for s in small])
    xs = np.ascontiguousarray(inputs.hidden(cfg, 0xAC, 16, tag="q"))
    d_x = L.kvl_mla_device_alloc(xs.nbytes)
    d_o = L.kvl_mla_device_alloc(xs.nbytes)
    lib.check(L.kvl_mla_copy_to_device(d_x, xs.ctypes.data, xs.nbytes), "h2d")
    # warm up (the RoPE table to 65,536 positions) and capture an allocating-path graph
    big = make_states(cfg, [40000] * 16, 0xC10)
    barr = (Q8P * 16)(*[C.pointer(s) for s in big])
    lib.check(L.kvl_mla_decode_compressed_q8_batch_device(d_o, d_x, 1, C.byref(cfg), C.byref(w), barr,
                                                          lib.NO_ADVANCE), "warm-up")
    lib.check(L.kvl_mla_decode_compressed_q8_batch_device(d_o, d_x, 2, C.byref(cfg), C.byref(w), sarr,
                                                          lib.NO_ADVANCE), "warm-up")
    lib.check(L.kvl_mla_synchronize(), "sync")
    lib.check(L.kvl_mla_capture_begin(), "capture begin")
    rc = L.kvl_mla_decode_compressed_q8_batch_device(d_o, d_x, 2, C.byref(cfg), C.byref(w), sarr, lib.NO_ADVANCE)
    g0 = C.c_void_p()
    lib.check(L.kvl_mla_capture_end(C.byref(g0)), "capture end")
    lib.check(rc, "captured allocating-path call")
    # 16 x 40,000 rows: 624 splits, more than any earlier call of this test made
    print("[noalloc] larger plan: 16 x 40000 rows", flush=True)
    nx = L.kvl_mla_decode_compressed_q8_batch_device_noalloc
    d_big = L.kvl_mla_device_alloc(xs.nbytes)
    lib.check(nx(d_big, d_x, 16, C.byref(cfg), C.byref(w), barr, lib.NO_ADVANCE), "no-allocation call, large plan")
    lib.check(L.kvl_mla_synchronize(), "sync")
    lib.check(L.kvl_mla_graph_launch(g0), "graph captured before the large no-allocation call")
    lib.check(L.kvl_mla_synchronize(), "sync")
    lib.check(L.kvl_mla_graph_destroy(g0), "graph destroy")
    # under capture
    print("[noalloc] captured no-allocation call, three replays", flush=True)
    lib.check(nx(d_o, d_x, 16, C.byref(cfg), C.byref(w), barr, lib.NO_ADVANCE), "eager")
    eager = np.zeros_like(xs)
    lib.check(L.kvl_mla_copy_to_host(eager.ctypes.data, d_o, xs.nbytes), "d2h")
    lib.check(L.kvl_mla_capture_begin(), "capture begin")
    rc = nx(d_o, d_x, 16, C.byref(cfg), C.byref(w), barr, lib.NO_ADVANCE)
    g1 = C.c_void_p()
    lib.check(L.kvl_mla_capture_end(C.byref(g1)), "capture end")
    lib.check(rc, "captured no-allocation call")
    for rep in range(3):
        junk = np.full_like(xs, 3.0)
        lib.check(L.kvl_mla_copy_to_device(d_o, junk.ctypes.data, xs.nbytes), "clear")
        lib.check(L.kvl_mla_graph_launch(g1), "graph launch")
        lib.check(L.kvl_mla_synchronize(), "sync")
        got = np.zeros_like(xs)
        lib.check(L.kvl_mla_copy_to_host(got.ctypes.data, d_o, xs.nbytes), "d2h")
        np.testing.assert_array_equal(got, eager, err_msg=f"replay {rep}")
        lib.check(nx(d_big, d_x, 2, C.byref(cfg), C.byref(w), sarr, lib.NO_ADVANCE), "eager between replays")
        lib.check(L.kvl_mla_synchronize(), "sync")
    lib.check(L.kvl_mla_graph_destroy(g1), "graph destroy")
    for p in (d_x, d_o, d_big):
        L.kvl_mla_device_free(p)
    for st in small + big:
        L.kvl_mla_compressed_q8_state_free(C.byref(st))
    L.kvl_mla_release_weights(C.byref(w))
