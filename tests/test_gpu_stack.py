"""The 27-layer decode workload that bench.py times, checked against the oracle.

27 layers, batch 8, a 32768-token row-wise Q8 latent history per layer and sequence
(device-generated), random-init bf16 weights, one decode token per sequence chained through
the layers with the residual add (KVL_MLA_RESIDUAL | KVL_MLA_NO_ADVANCE, as bench.py calls
it). The attention splits here are the production plan: 256 workgroups of ~1024 rows.

The layer outputs h_{l+1} - h_l of layers 0 and 26 are compared with the oracle's decode
(src/mla_compressed_q8_state.c:161-255, the reference's arithmetic in double) of the same
input h_l over that layer's rows, pulled back from the device, for two sequences each:
max|got - ref| / max|ref| <= 2e-3. The chain is then captured in a HIP graph and replayed;
the replays reproduce the eager chain bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import Api, f32, rel_err
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

TOL = 2e-3
L = lib.load()
O = Api(pyoracle.load_oracle(), "orc_")


def test_stack_27_layers_batch8_32k_q8_vs_oracle():
    NL, B, CTX = 27, 8, 32768
    cfg = inputs.config(**inputs.KIMI)
    H = cfg.hidden_size
    print(f"[stack] {NL} layers, batch {B}, {CTX}-token Q8 histories", flush=True)
    layers = [inputs.fast_layer(cfg, 0xC4 + li) for li in range(NL)]
    ws = [ly.struct() for ly in layers]
    for w in ws:
        lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    Q8P = C.POINTER(abi.KvlMlaCompressedQ8State)
    states, arrays = [], []
    for li in range(NL):
        row = []
        for b in range(B):
            st = abi.KvlMlaCompressedQ8State()
            assert L.kvl_mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), CTX + 1) == 0
            lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, CTX, inputs.stack_seed(li, b)),
                      "fill")
            row.append(st)
        states.append(row)
        arrays.append((Q8P * B)(*[C.pointer(s) for s in row]))
    print("[stack]   histories generated", flush=True)
    x0 = np.ascontiguousarray(inputs.hidden(cfg, 0xC4, B, tag="stack_x"))
    nbytes = x0.nbytes
    d_x0, d_h = L.kvl_mla_device_alloc(nbytes), L.kvl_mla_device_alloc(nbytes)
    assert d_x0 and d_h
    lib.check(L.kvl_mla_copy_to_device(d_x0, x0.ctypes.data, nbytes), "h2d")
    flags = lib.RESIDUAL | lib.NO_ADVANCE
    checked = (0, NL - 1)
    hs = {}

    def pull():
        h = np.zeros_like(x0)
        lib.check(L.kvl_mla_copy_to_host(h.ctypes.data, d_h, nbytes), "d2h")
        return h

    def chain(record):
        lib.check(L.kvl_mla_copy_kernel(d_h, d_x0, nbytes), "reset hidden")
        for li in range(NL):
            if record and (li in checked or li - 1 in checked):
                lib.check(L.kvl_mla_synchronize(), "sync")
                hs[li] = pull()
            lib.check(L.kvl_mla_decode_compressed_q8_batch_device(d_h, d_h, B, C.byref(cfg), C.byref(ws[li]),
                                                                  arrays[li], flags), f"layer {li}")

    chain(True)
    lib.check(L.kvl_mla_synchronize(), "sync")
    hs[NL] = pull()
    assert np.all(np.isfinite(hs[NL]))
    print("[stack]   eager chain done", flush=True)

    for li in checked:
        for b in (0, 5):
            st = states[li][b]
            lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, CTX), "pull rows")
            ref = np.zeros(H, np.float32)
            x = np.ascontiguousarray(hs[li][b])
            assert O.mla_decode_compressed_q8_bf16(f32(ref), f32(x), CTX, C.byref(cfg), C.byref(ws[li]),
                                                   C.byref(st)) == 0
            st.len = CTX  # the oracle appended at position CTX; the device copy holds rows [0, CTX)
            got = hs[li + 1][b].astype(np.float64) - hs[li][b].astype(np.float64)
            e = rel_err(got, ref)
            print(f"[stack]   layer {li} sequence {b}: max|d|/max|ref| = {e:.3e}", flush=True)
            assert e <= TOL, (li, b, e)

    # the same chain as a HIP graph (the benchmark's timed form), replayed with eager work between
    lib.check(L.kvl_mla_capture_begin(), "capture begin")
    try:
        chain(False)
    finally:
        ge = C.c_void_p()
        rc = L.kvl_mla_capture_end(C.byref(ge))
    lib.check(rc, "capture end")
    junk = np.full_like(x0, 7.0)
    for rep in range(2):
        lib.check(L.kvl_mla_copy_to_device(d_h, junk.ctypes.data, nbytes), "scramble")
        lib.check(L.kvl_mla_graph_launch(ge), "graph launch")
        lib.check(L.kvl_mla_synchronize(), "sync")
        np.testing.assert_array_equal(pull(), hs[NL], err_msg=f"replay {rep}")
    lib.check(L.kvl_mla_graph_destroy(ge), "graph destroy")
    L.kvl_mla_device_free(d_x0)
    L.kvl_mla_device_free(d_h)
    for row in states:
        for st in row:
            L.kvl_mla_compressed_q8_state_free(C.byref(st))
    for w in ws:
        L.kvl_mla_release_weights(C.byref(w))
