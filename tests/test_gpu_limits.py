"""Limits of the device path: many long sequences in one batched call (more split-K partials
than one sequence may have), graph replays after the library's buffers moved, and the generic
prefill route at a length where its score scratch is tiled over queries."""
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
Q8P = C.POINTER(abi.KvlMlaCompressedQ8State)


def q8_states(cfg, lens, seed):
    sts = []
    for i, n in enumerate(lens):
        st = abi.KvlMlaCompressedQ8State()
        assert L.kvl_mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), int(n) + 1) == 0
        lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, int(n), seed + i), "fill")
        sts.append(st)
    return sts


def test_q8_batch_with_more_than_2048_splits():
    """64 sequences of ~40K rows: the launch has ~2500 split-K partials (about 39 per sequence,
    so each sequence stays within the combine's limit). Batched outputs against lone decodes
    of the same tokens, and two sequences against the oracle."""
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.make_layer(cfg, 0xF1)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    rng = np.random.default_rng(0xF1)
    lens = rng.integers(39000, 41000, size=64)
    B, H = len(lens), cfg.hidden_size
    print(f"[limits] 64 Q8 sequences, {int(lens.sum())} rows", flush=True)
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xF1, B, tag="q"))
    sts = q8_states(cfg, lens, 0xF100)
    arr = (Q8P * B)(*[C.pointer(s) for s in sts])
    pos = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.zeros((B, H), np.float32)
    lib.check(L.kvl_mla_decode_compressed_q8_batch_bf16(f32(out), f32(xb), pos.ctypes.data_as(C.POINTER(C.c_int)), B,
                                                        C.byref(cfg), C.byref(w), arr), "batched decode")
    for s in sts:
        L.kvl_mla_compressed_q8_state_free(C.byref(s))
    lone_sts = q8_states(cfg, lens, 0xF100)
    worst = 0.0
    for i, st in enumerate(lone_sts):
        o = np.zeros(H, np.float32)
        lib.check(L.kvl_mla_decode_compressed_q8_bf16(f32(o), f32(xb[i]), int(lens[i]), C.byref(cfg), C.byref(w),
                                                      C.byref(st)), f"lone {i}")
        worst = max(worst, rel_err(out[i], o))
    print(f"[limits]   batch vs lone max rel err {worst:.3e}", flush=True)
    assert worst <= 1e-4
    for i in (0, 63):
        st = lone_sts[i]
        n = int(lens[i])
        lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, n), "pull")
        st.len = n
        ref = np.zeros(H, np.float32)
        assert O.mla_decode_compressed_q8_bf16(f32(ref), f32(xb[i]), n, C.byref(cfg), C.byref(w), C.byref(st)) == 0
        e = rel_err(out[i], ref)
        print(f"[limits]   sequence {i} ({n} rows) vs oracle {e:.3e}", flush=True)
        assert e <= TOL
    for s in lone_sts:
        L.kvl_mla_compressed_q8_state_free(C.byref(s))
    L.kvl_mla_release_weights(C.byref(w))


def test_graph_refused_after_buffers_moved():
    """A captured graph keeps working while nothing moves; once library device memory is
    released (here: freeing a state, whose device copy goes away), the old graph is refused
    (-1, with a reason) instead of replaying on possibly freed memory, and a new capture works.
    Workspace growth and RoPE-table growth release memory the same way."""
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.make_layer(cfg, 0xF2)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    sts = q8_states(cfg, [3000, 2500, 1000], 0xF200)
    x = np.ascontiguousarray(inputs.hidden(cfg, 0xF2, 2, tag="q"))
    dx, do = L.kvl_mla_device_alloc(x.nbytes), L.kvl_mla_device_alloc(x.nbytes)
    lib.check(L.kvl_mla_copy_to_device(dx, x.ctypes.data, x.nbytes), "h2d")
    arr2 = (Q8P * 2)(*[C.pointer(s) for s in sts[:2]])
    dec = L.kvl_mla_decode_compressed_q8_batch_device
    lib.check(dec(do, dx, 2, C.byref(cfg), C.byref(w), arr2, lib.NO_ADVANCE), "warm")

    def capture():
        lib.check(L.kvl_mla_capture_begin(), "capture")
        rc = dec(do, dx, 2, C.byref(cfg), C.byref(w), arr2, lib.NO_ADVANCE)
        ge = C.c_void_p()
        lib.check(L.kvl_mla_capture_end(C.byref(ge)), "capture end")
        lib.check(rc, "captured decode")
        return ge

    ge = capture()
    for _ in range(2):
        lib.check(L.kvl_mla_graph_launch(ge), "replay")
        lib.check(L.kvl_mla_synchronize(), "sync")
    L.kvl_mla_compressed_q8_state_free(C.byref(sts[2]))  # releases that state's device copy
    assert L.kvl_mla_graph_launch(ge) == -1
    assert "capture it again" in lib.last_error()
    lib.check(L.kvl_mla_graph_destroy(ge), "destroy")
    ge = capture()
    lib.check(L.kvl_mla_graph_launch(ge), "replay of the new capture")
    lib.check(L.kvl_mla_synchronize(), "sync")
    lib.check(L.kvl_mla_graph_destroy(ge), "destroy")
    L.kvl_mla_device_free(dx)
    L.kvl_mla_device_free(do)
    for s in sts[:2]:
        L.kvl_mla_compressed_q8_state_free(C.byref(s))
    L.kvl_mla_release_weights(C.byref(w))


def test_generic_prefill_tiled_queries():
    """Shapes outside the MFMA route (the streaming probe's, src/mla_streaming_probe.c:39,46)
    at 3000 tokens: the score scratch is tiled over queries (the whole S x NH x S matrix would
    exceed the 64 MiB tile), and the result matches the oracle's streaming prefill."""
    dims = dict(hidden_size=16, num_heads=2, qk_nope_dim=4, qk_rope_dim=4, v_head_dim=8, kv_lora_rank=6,
                rms_eps=1e-5, rope_theta=800000.0)
    cfg = inputs.config(**dims)
    layer = inputs.make_layer(cfg, 0xF3, std=0.2)
    S = 3000
    x = (inputs.hidden(cfg, 0xF3, S) * np.float32(0.25)).astype(np.float32)
    w = layer.struct()
    a = np.zeros((S, 16), np.float32)
    b = np.zeros((S, 16), np.float32)
    lib.check(L.kvl_mla_prefill_bf16(f32(a), f32(x), S, C.byref(cfg), C.byref(w)), "prefill")
    assert O.lib.orc_mla_prefill_streaming(f32(b), f32(x), S, C.byref(cfg), C.byref(w)) == 0
    e = rel_err(a, b)
    print(f"[limits] generic prefill S={S} vs oracle {e:.3e}", flush=True)
    assert e <= TOL
