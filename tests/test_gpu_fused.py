"""The Q8 decode of two or more independent sequences prepares the queries and appends the rows
inside its attention launch (the launch's lowest-numbered workgroups work for the others, which
wait for them on device flags); kvl_mla_set_fused_qprep(0) selects the two-launch form
(k_append_qprep, then the attention). Both forms must give the same outputs, the same appended
rows and the same states bit for bit (the parity of the two-launch form with the oracle is
tested elsewhere, and the block decode, which always takes it, equals single decodes bit for
bit). The cases cover the fused form's edges: eight long sequences (one round of workgroups),
short sequences whose single split holds the new row in its first chunks (their requests wait
for the append inside the prologue) beside long ones, and two consecutive steps (the flags are
cleared by each step's projection launch). For eight sequences with equal split counts the fused
launch also combines the split partials (kvl_mla_set_fused_combine; each sequence's splits on one
XCD): that form must equal the others bit for bit as well, with fewer splits than combine tasks
(six thousand rows: 24 splits, so a workgroup takes two tasks). With at least 232 splits for at
most eight sequences the launch also computes the q_proj | kv_a projection
(kvl_mla_set_fused_projection): eight sequences of 8000 rows (256 splits: projection and
combine) and three sequences of 63, 30000 and 30000 rows (237 splits: projection only) cover it;
every combination of the switches must give the same bits. Sequences of 16 or more splits each
combine across XCDs (their partials stored past the L2s): a lone sequence of 9000 rows (64
splits; the fused form of a lone sequence needs the projection and the combine inside the
launch, so with either switch off it takes the two-launch form), a lone sequence of 2100 rows
(17 splits, the fewest the fused form takes: 15 of its workgroups combine two (head, half)
pairs) and two of 20000 and 30000 rows (79 + 118 splits)."""
import ctypes as C

import numpy as np
import pytest

from helpers import f32
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

L = lib.load()
KIMI = dict(inputs.KIMI)

# history rows per sequence; each case needs 17 x batch <= the launch's split count
CASES = [(6000,) * 8, (100, 9000), (9000, 200, 130, 9000), (63, 9000, 9000), (8000,) * 8, (63, 30000, 30000),
         (9000,), (20000, 30000), (2100,)]


def switches(form, comb, proj):
    prev = (L.kvl_mla_set_fused_qprep(form), L.kvl_mla_set_fused_combine(comb), L.kvl_mla_set_fused_projection(proj))
    assert all(p in (0, 1) for p in prev), prev
    return prev


def restore(prev):
    L.kvl_mla_set_fused_qprep(prev[0])
    L.kvl_mla_set_fused_combine(prev[1])
    L.kvl_mla_set_fused_projection(prev[2])


def run(form, lens, cfg, w, x, steps, comb=1, proj=1):
    prev = switches(form, comb, proj)
    try:
        states = []
        for i, n in enumerate(lens):
            st = abi.KvlMlaCompressedQ8State()
            lib.check(L.kvl_mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), n + steps), "init")
            lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, n, 0xF00 + i), "fill")
            lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, n), "pull")
            states.append(st)
        arr = (C.POINTER(abi.KvlMlaCompressedQ8State) * len(lens))(*[C.pointer(s) for s in states])
        outs = []
        for t in range(steps):
            pos = np.ascontiguousarray([n + t for n in lens], dtype=np.int32)
            out = np.zeros((len(lens), cfg.hidden_size), np.float32)
            lib.check(L.kvl_mla_decode_compressed_q8_batch_bf16(f32(out), f32(np.ascontiguousarray(x[t])),
                                                                pos.ctypes.data_as(C.POINTER(C.c_int)), len(lens),
                                                                C.byref(cfg), C.byref(w), arr), f"step {t}")
            outs.append(out)
        rows = []
        R, DR = cfg.kv_lora_rank, cfg.qk_rope_dim
        for st, n in zip(states, lens):
            m = n + steps
            assert st.len == m
            rows.append((np.ctypeslib.as_array(st.latent_q8, (m * R,)).copy(),
                         np.ctypeslib.as_array(st.latent_scale, (m,)).copy(),
                         np.ctypeslib.as_array(st.rope_bf16, (m * DR,)).copy()))
        for st in states:
            L.kvl_mla_compressed_q8_state_free(C.byref(st))
        return outs, rows
    finally:
        restore(prev)


@pytest.mark.parametrize("lens", CASES, ids=["-".join(map(str, c)) for c in CASES])
def test_fused_equals_two_launch_form(lens):
    print(f"[fused] lens {lens}", flush=True)
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xF1)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    try:
        steps = 2
        x = np.stack([inputs.hidden(cfg, 0xF2 + t, len(lens)) for t in range(steps)])
        so, sr = run(0, lens, cfg, w, x, steps)
        for comb, proj in ((1, 1), (1, 0), (0, 1), (0, 0)):
            fo, fr = run(1, lens, cfg, w, x, steps, comb=comb, proj=proj)
            form = f"fused, combine {comb}, projection {proj}"
            for t in range(steps):
                assert np.isfinite(fo[t]).all()
                np.testing.assert_array_equal(fo[t], so[t], err_msg=f"step {t} outputs ({form})")
            for i in range(len(lens)):
                for k, name in enumerate(("codes", "scales", "rope")):
                    np.testing.assert_array_equal(fr[i][k], sr[i][k], err_msg=f"sequence {i} {name} ({form})")
    finally:
        L.kvl_mla_release_weights(C.byref(w))


def test_fused_switch_rejects_bad_values():
    prev = L.kvl_mla_set_fused_qprep(1)
    assert prev in (0, 1)
    assert L.kvl_mla_set_fused_qprep(2) == -1
    assert L.kvl_mla_set_fused_qprep(prev) == 1
    prev = L.kvl_mla_set_fused_combine(1)
    assert prev in (0, 1)
    assert L.kvl_mla_set_fused_combine(-1) == -1
    assert L.kvl_mla_set_fused_combine(prev) == 1
    prev = L.kvl_mla_set_fused_projection(1)
    assert prev in (0, 1)
    assert L.kvl_mla_set_fused_projection(3) == -1
    assert L.kvl_mla_set_fused_projection(prev) == 1


def test_fused_wait_timeout_is_reported_and_recovered():
    """The failure path, forced from the host: with the fused launch's wait bound at one tick of
    the 100 MHz counter its waits end before the work they wait for is done (every kernel still
    runs to its end). The host-buffer call returns -1 with the timeout message and leaves the
    states as they were; a stream-ordered call is reported by kvl_mla_synchronize. With the
    default bound the next calls equal the two-launch form bit for bit (the flags left behind
    are cleared)."""
    print("[fused] forced wait timeouts, 8 x 8000 rows", flush=True)
    lens = (8000,) * 8
    cfg = inputs.config(**KIMI)
    layer = inputs.make_layer(cfg, 0xF6)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    x = np.stack([inputs.hidden(cfg, 0xF7, len(lens))])
    so, sr = run(0, lens, cfg, w, x, 1)
    prev = switches(1, 1, 1)
    states = []
    d_x = d_o = None
    try:
        for i, n in enumerate(lens):
            st = abi.KvlMlaCompressedQ8State()
            lib.check(L.kvl_mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), n + 1), "init")
            lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, n, 0xF00 + i), "fill")
            lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, n), "pull")
            states.append(st)
        arr = (C.POINTER(abi.KvlMlaCompressedQ8State) * len(lens))(*[C.pointer(s) for s in states])
        pos = np.ascontiguousarray(lens, dtype=np.int32)
        xs = np.ascontiguousarray(x[0])
        out = np.zeros((len(lens), cfg.hidden_size), np.float32)

        def call():
            return L.kvl_mla_decode_compressed_q8_batch_bf16(f32(out), f32(xs), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                                             len(lens), C.byref(cfg), C.byref(w), arr)

        # host-buffer call
        assert L.kvl_mla_set_fused_wait_limit(1) == 0
        assert call() == -1
        assert "timed out" in lib.last_error()
        assert [s.len for s in states] == list(lens)
        # stream-ordered call: enqueued, reported at the synchronisation
        d_x = L.kvl_mla_device_alloc(xs.nbytes)
        d_o = L.kvl_mla_device_alloc(out.nbytes)
        assert d_x and d_o
        lib.check(L.kvl_mla_copy_to_device(d_x, xs.ctypes.data, xs.nbytes), "h2d")
        rc = L.kvl_mla_decode_compressed_q8_batch_device(d_o, d_x, len(lens), C.byref(cfg), C.byref(w), arr,
                                                         lib.NO_ADVANCE)
        assert rc == 0, lib.last_error()
        assert L.kvl_mla_synchronize() == -1
        assert "timed out" in lib.last_error()
        # default bound: normal results again
        assert L.kvl_mla_set_fused_wait_limit(0) == 0
        rc = L.kvl_mla_decode_compressed_q8_batch_device(d_o, d_x, len(lens), C.byref(cfg), C.byref(w), arr,
                                                         lib.NO_ADVANCE)
        assert rc == 0, lib.last_error()
        assert L.kvl_mla_synchronize() == 0, lib.last_error()
        lib.check(call(), "host call after the timeouts")
        np.testing.assert_array_equal(out, so[0], err_msg="outputs after the timeouts")
        R, DR = cfg.kv_lora_rank, cfg.qk_rope_dim
        for i, (st, n) in enumerate(zip(states, lens)):
            m = n + 1
            assert st.len == m
            np.testing.assert_array_equal(np.ctypeslib.as_array(st.latent_q8, (m * R,)), sr[i][0])
            np.testing.assert_array_equal(np.ctypeslib.as_array(st.latent_scale, (m,)), sr[i][1])
            np.testing.assert_array_equal(np.ctypeslib.as_array(st.rope_bf16, (m * DR,)), sr[i][2])
    finally:
        L.kvl_mla_set_fused_wait_limit(0)
        restore(prev)
        if d_x:
            L.kvl_mla_device_free(d_x)
        if d_o:
            L.kvl_mla_device_free(d_o)
        for st in states:
            L.kvl_mla_compressed_q8_state_free(C.byref(st))
        L.kvl_mla_release_weights(C.byref(w))
