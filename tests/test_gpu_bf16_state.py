"""The BF16-latent state (include/kvl/mla_hip.h) on the GPU, against the oracle's FP32 decode
(src/mla_compressed_state.c:86-161) over the same bf16-valued history.

The oracle side is an FP32 state whose rows [0, t) are set, before each decode, to the BF16
state's rows converted to fp32 (exact), decoded by orc_mla_decode_compressed_bf16_rows: the FP32
decode with its appended row rounded to bf16 as the state stores it (pinned in test_oracle.py).
Bars:
  - stored rows: the bf16 round-to-nearest-even of the oracle's fp32 rows, except where the
    projection's summation order moves the fp32 value across a rounding boundary (under 1 % of
    the elements, each within one bf16 step plus 1e-5 of its row's largest element);
  - attention outputs: max|got - ref| / max|ref| <= 2e-3;
  - block decode and batched decode: bit-identical / 1e-4 against single-token decodes.
"""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import Api, f32, rel_err
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

TOL = 2e-3
O = Api(pyoracle.load_oracle(), "orc_")
L = lib.load()
G = Api(L, "kvl_")
BSP = C.POINTER(abi.KvlMlaCompressedBF16State)

TINY = dict(hidden_size=16, num_heads=2, qk_nope_dim=4, qk_rope_dim=4, v_head_dim=4,
            kv_lora_rank=6, rms_eps=1e-6, rope_theta=10000.0)
LAB = dict(hidden_size=64, num_heads=4, qk_nope_dim=8, qk_rope_dim=8, v_head_dim=8,
           kv_lora_rank=32, rms_eps=1e-6, rope_theta=10000.0)
KIMI = dict(inputs.KIMI)


def model(d, seed, std=0.02, n=8, q_std=None):
    cfg = inputs.config(**d)
    layer = inputs.make_layer(cfg, seed, std=std, q_std=q_std)
    return cfg, layer, np.ascontiguousarray(inputs.hidden(cfg, seed, n))


def new_bf16(cfg, cap):
    st = abi.KvlMlaCompressedBF16State()
    lib.check(L.kvl_mla_compressed_bf16_state_init(C.byref(st), C.byref(cfg), int(cap)), "bf16 init")
    return st


def rows_of(st, n):
    """Host rows [0, n) of a BF16 state: (latent bits [n, R], rope bits [n, DR])."""
    R, DR = st.kv_lora_rank, st.qk_rope_dim
    lat = np.ctypeslib.as_array(st.latent, (st.capacity * R,))[:n * R].reshape(n, R).copy()
    rope = np.ctypeslib.as_array(st.rope, (st.capacity * DR,))[:n * DR].reshape(n, DR).copy()
    return lat, rope


def new_twin(cfg, cap):
    st = abi.KvlMlaCompressedState()
    assert O.mla_compressed_state_init(C.byref(st), C.byref(cfg), int(cap)) == 0
    return st


def set_twin(twin, bst, n):
    """The oracle FP32 state holds the BF16 state's rows [0, n) as fp32 values; len = n."""
    R, DR = bst.kv_lora_rank, bst.qk_rope_dim
    lat, rope = rows_of(bst, n)
    np.ctypeslib.as_array(twin.latent, (twin.capacity * R,))[:n * R] = inputs.bf16_bits_to_f32(lat).ravel()
    np.ctypeslib.as_array(twin.rope, (twin.capacity * DR,))[:n * DR] = inputs.bf16_bits_to_f32(rope).ravel()
    twin.len = n


def assert_rows_round(bits, ref_f32, what):
    """bf16 rows are the RNE rounding of the oracle's fp32 rows: equal codes in >= 99 % of the
    elements; elsewhere the fp32 values differ by the projection's summation order, so the code
    stays within one bf16 step (2^-7 relative) plus 1e-5 of the row's largest element."""
    ref = np.ascontiguousarray(ref_f32, dtype=np.float32)
    want = inputs.f32_to_bf16_bits(ref)
    miss = bits != want
    got = inputs.bf16_bits_to_f32(bits).astype(np.float64)
    r64 = ref.astype(np.float64)
    bound = np.abs(r64) * 2.0 ** -7 + 1e-5 * np.max(np.abs(r64), axis=-1, keepdims=True)
    assert miss.mean() < 0.01 and np.all(np.abs(got - r64) <= bound), (what, float(miss.mean()))


def oracle_decode(cfg, w, twin, bst, x, pos):
    set_twin(twin, bst, pos)
    ref = np.zeros(cfg.hidden_size, np.float32)
    assert O.mla_decode_compressed_bf16_rows(f32(ref), f32(x), pos, C.byref(cfg), C.byref(w), C.byref(twin)) == 0
    return ref, np.asarray(np.ctypeslib.as_array(twin.latent, (twin.capacity * cfg.kv_lora_rank,))
                           [pos * cfg.kv_lora_rank:(pos + 1) * cfg.kv_lora_rank]).copy()


SHAPES = [("tiny", TINY, 0.2, 9, 4), ("lab", LAB, 0.05, 13, 6), ("kimi", KIMI, 0.02, 40, 24)]


@pytest.mark.parametrize("name,dims,std,S,P", SHAPES, ids=[s[0] for s in SHAPES])
def test_prefill_and_decode_match_oracle(name, dims, std, S, P):
    """State prefill of P tokens, then one decode per remaining token. Generic kernels for the
    probe shapes, the bf16 MFMA kernel for the Kimi shapes."""
    print(f"[bf16] shape={name} S={S} prefill={P}", flush=True)
    cfg, layer, x = model(dims, 0xB1, std=std, n=S)
    w = layer.struct()
    st = new_bf16(cfg, S + 1)
    lib.check(L.kvl_mla_compressed_bf16_state_prefill_bf16(f32(x[:P]), P, C.byref(cfg), C.byref(w), C.byref(st)),
              "bf16 prefill")
    assert st.len == P
    ref_st = new_twin(cfg, S + 1)
    assert O.mla_compressed_state_prefill_bf16(f32(x[:P]), P, C.byref(cfg), C.byref(w), C.byref(ref_st)) == 0
    lat, rope = rows_of(st, P)
    R, DR = cfg.kv_lora_rank, cfg.qk_rope_dim
    assert_rows_round(lat, np.ctypeslib.as_array(ref_st.latent, (ref_st.capacity * R,))[:P * R].reshape(P, R), "latent")
    assert_rows_round(rope, np.ctypeslib.as_array(ref_st.rope, (ref_st.capacity * DR,))[:P * DR].reshape(P, DR), "rope")
    twin = new_twin(cfg, S + 1)
    worst = 0.0
    for t in range(P, S):
        got = np.zeros(cfg.hidden_size, np.float32)
        lib.check(L.kvl_mla_decode_compressed_bf16_bf16(f32(got), f32(x[t]), t, C.byref(cfg), C.byref(w),
                                                         C.byref(st)), f"decode {t}")
        assert st.len == t + 1
        ref, ref_row = oracle_decode(cfg, w, twin, st, x[t], t)
        worst = max(worst, rel_err(got, ref))
        assert_rows_round(rows_of(st, t + 1)[0][t:t + 1], ref_row[None], f"row {t}")
    print(f"[bf16]   worst max|d|/max|ref| = {worst:.3e}", flush=True)
    assert worst <= TOL
    for s in (st,):
        L.kvl_mla_compressed_bf16_state_free(C.byref(s))
    for s in (ref_st, twin):
        O.mla_compressed_state_free(C.byref(s))


@pytest.mark.parametrize("n", [8192, 32768])
def test_long_history_sharp_logits(n):
    """Large attention logits (q_proj std 8x) over a long history of random bf16 rows: many
    32-row chunks per split, moving maxima inside a split and across splits."""
    cfg, layer, _ = model(KIMI, 0xB2, q_std=0.16)
    w = layer.struct()
    lat = inputs.normal_f32(0xB2, "lat", (n, 512))
    rope = inputs.normal_f32(0xB2, "rope", (n, 64))
    st = new_bf16(cfg, n + 1)
    np.ctypeslib.as_array(st.latent, ((n + 1) * 512,))[:n * 512] = inputs.f32_to_bf16_bits(lat).ravel()
    np.ctypeslib.as_array(st.rope, ((n + 1) * 64,))[:n * 64] = inputs.f32_to_bf16_bits(rope).ravel()
    st.len = n
    x = inputs.hidden(cfg, 0xB2, 1, tag="query")[0]
    got = np.zeros(cfg.hidden_size, np.float32)
    lib.check(L.kvl_mla_decode_compressed_bf16_bf16(f32(got), f32(x), n, C.byref(cfg), C.byref(w), C.byref(st)),
              "decode")
    twin = new_twin(cfg, n + 1)
    ref, _ = oracle_decode(cfg, w, twin, st, x, n)
    e = rel_err(got, ref)
    print(f"[bf16] {n} rows, sharp logits: max|d|/max|ref| = {e:.3e}", flush=True)
    assert e <= TOL
    L.kvl_mla_compressed_bf16_state_free(C.byref(st))
    O.mla_compressed_state_free(C.byref(twin))


def test_ragged_batch_with_partial_chunks():
    """One batched call over histories of 0, 1, 31, 32, 33, 127, 128, 129, 1000 and 5001 rows
    (partial last chunks, a lone 32-row chunk, the shortest split), each against the oracle."""
    cfg, layer, _ = model(KIMI, 0xB3)
    w = layer.struct()
    lens = [0, 1, 31, 32, 33, 127, 128, 129, 1000, 5001]
    B = len(lens)
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xB3, B, tag="query"))
    sts = []
    for i, n in enumerate(lens):
        st = new_bf16(cfg, n + 1)
        if n:
            lib.check(L.kvl_mla_compressed_bf16_state_fill_synthetic(C.byref(st), 0, n, 0xB30 + i), "fill")
            lib.check(L.kvl_mla_compressed_bf16_state_pull(C.byref(st), 0, n), "pull")
        sts.append(st)
    arr = (BSP * B)(*[C.pointer(s) for s in sts])
    pos = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.zeros((B, cfg.hidden_size), np.float32)
    lib.check(L.kvl_mla_decode_compressed_bf16_batch_bf16(f32(out), f32(xb), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                                          B, C.byref(cfg), C.byref(w), arr), "batched decode")
    twin = new_twin(cfg, max(lens) + 1)
    for i, n in enumerate(lens):
        assert sts[i].len == n + 1
        ref, ref_row = oracle_decode(cfg, w, twin, sts[i], xb[i], n)
        e = rel_err(out[i], ref)
        assert e <= TOL, (n, e)
        assert_rows_round(rows_of(sts[i], n + 1)[0][n:n + 1], ref_row[None], f"row {n}")
    for s in sts:
        L.kvl_mla_compressed_bf16_state_free(C.byref(s))
    O.mla_compressed_state_free(C.byref(twin))


def test_config2_ragged_64_sequences_bf16_state():
    """64 sequences, context lengths uniform in [512, 32768] (seeded), each with its own BF16
    latent cache (1152 B per row, device-generated), one query each, through the batched entry
    point. Every sequence against a lone decode of the same token (the batch only moves the
    split boundaries), and 6 of them (shortest, longest, 4 others) against the oracle."""
    cfg, layer, _ = model(KIMI, 0xC8)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    rng = np.random.default_rng(0xC8)
    lens = rng.integers(512, 32769, size=64)
    B, H = len(lens), cfg.hidden_size
    print(f"[bf16 config2] 64 sequences, {int(lens.sum())} rows", flush=True)
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xC8, B, tag="query"))

    def make_states():
        sts = []
        for i, n in enumerate(lens):
            st = new_bf16(cfg, int(n) + 1)
            lib.check(L.kvl_mla_compressed_bf16_state_fill_synthetic(C.byref(st), 0, int(n), 0xC80 + i), "fill")
            sts.append(st)
        return sts

    batch_states = make_states()
    arr = (BSP * B)(*[C.pointer(s) for s in batch_states])
    pos = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.zeros((B, H), np.float32)
    lib.check(L.kvl_mla_decode_compressed_bf16_batch_bf16(f32(out), f32(xb), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                                          B, C.byref(cfg), C.byref(w), arr), "batched decode")
    assert all(s.len == n + 1 for s, n in zip(batch_states, lens))
    for s in batch_states:
        L.kvl_mla_compressed_bf16_state_free(C.byref(s))
    print("[bf16 config2]   batch done; lone decodes", flush=True)
    lone_states = make_states()
    lone = np.zeros_like(out)
    for i, st in enumerate(lone_states):
        lib.check(L.kvl_mla_decode_compressed_bf16_bf16(f32(lone[i]), f32(xb[i]), int(lens[i]), C.byref(cfg),
                                                         C.byref(w), C.byref(st)), f"lone decode {i}")
    worst = max(rel_err(out[i], lone[i]) for i in range(B))
    print(f"[bf16 config2]   batch vs lone max rel err {worst:.3e}", flush=True)
    assert worst <= 1e-4
    twin = new_twin(cfg, int(lens.max()) + 1)
    for i in sorted({int(np.argmin(lens)), int(np.argmax(lens)), 5, 17, 33, 50}):
        st = lone_states[i]
        n = int(lens[i])
        lib.check(L.kvl_mla_compressed_bf16_state_pull(C.byref(st), 0, n), "pull")
        ref, _ = oracle_decode(cfg, w, twin, st, xb[i], n)
        e = rel_err(out[i], ref)
        print(f"[bf16 config2]   sequence {i} ({n} rows) vs oracle {e:.3e}", flush=True)
        assert e <= TOL, (i, n, e)
    for s in lone_states:
        L.kvl_mla_compressed_bf16_state_free(C.byref(s))
    O.mla_compressed_state_free(C.byref(twin))
    L.kvl_mla_release_weights(C.byref(w))


def test_block_equals_serial_and_oracle_block():
    """Block decode of 8 tokens after a 20000-row history == 8 single-token decodes bit for bit
    (outputs and stored rows), and within 2e-3 of the oracle's block decode over the same
    history (src/mla_compressed_state.c:163-184: the single-token decode in a loop)."""
    cfg, layer, _ = model(KIMI, 0xB4)
    w = layer.struct()
    n, T, H = 20000, 8, cfg.hidden_size
    x = np.ascontiguousarray(inputs.hidden(cfg, 0xB4, T, tag="draft"))
    outs, rows = [], []
    for mode in ("block", "serial"):
        st = new_bf16(cfg, n + T)
        lib.check(L.kvl_mla_compressed_bf16_state_fill_synthetic(C.byref(st), 0, n, 0xB40), "fill")
        lib.check(L.kvl_mla_compressed_bf16_state_pull(C.byref(st), 0, n), "pull")
        o = np.zeros((T, H), np.float32)
        if mode == "block":
            lib.check(L.kvl_mla_decode_compressed_bf16_block_bf16(f32(o), f32(x), T, n, C.byref(cfg), C.byref(w),
                                                                   C.byref(st)), "block")
        else:
            for t in range(T):
                lib.check(L.kvl_mla_decode_compressed_bf16_bf16(f32(o[t]), f32(x[t]), n + t, C.byref(cfg),
                                                                 C.byref(w), C.byref(st)), f"serial {t}")
        assert st.len == n + T
        outs.append(o)
        rows.append(rows_of(st, n + T))
        if mode == "block":
            twin = new_twin(cfg, n + T)
            set_twin(twin, st, n)
            ref = np.zeros((T, H), np.float32)
            for t in range(T):
                assert O.mla_decode_compressed_bf16_rows(f32(ref[t]), f32(x[t]), n + t, C.byref(cfg), C.byref(w),
                                                         C.byref(twin)) == 0
            e = rel_err(o, ref)
            print(f"[bf16] block of {T} at {n} rows vs oracle block {e:.3e}", flush=True)
            assert e <= TOL
            O.mla_compressed_state_free(C.byref(twin))
        L.kvl_mla_compressed_bf16_state_free(C.byref(st))
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(rows[0][0], rows[1][0])
    np.testing.assert_array_equal(rows[0][1], rows[1][1])


def test_device_api_graph_replay_and_truncate():
    """Batched device decode (KVL_MLA_NO_ADVANCE) eager and as three graph replays == the host
    API's outputs; truncate + re-decode == the first decode."""
    cfg, layer, _ = model(KIMI, 0xB5)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    lens = [3000, 4100, 700, 12345]
    B, H = len(lens), cfg.hidden_size
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xB5, B, tag="query"))
    sts = []
    for i, n in enumerate(lens):
        st = new_bf16(cfg, n + 2)
        lib.check(L.kvl_mla_compressed_bf16_state_fill_synthetic(C.byref(st), 0, n, 0xB50 + i), "fill")
        sts.append(st)
    arr = (BSP * B)(*[C.pointer(s) for s in sts])
    dx, do = L.kvl_mla_device_alloc(xb.nbytes), L.kvl_mla_device_alloc(xb.nbytes)
    lib.check(L.kvl_mla_copy_to_device(dx, xb.ctypes.data, xb.nbytes), "h2d")
    dec = L.kvl_mla_decode_compressed_bf16_batch_device
    lib.check(dec(do, dx, B, C.byref(cfg), C.byref(w), arr, lib.NO_ADVANCE), "eager device decode")
    eager = np.zeros((B, H), np.float32)
    lib.check(L.kvl_mla_copy_to_host(eager.ctypes.data, do, eager.nbytes), "d2h")
    assert [s.len for s in sts] == lens
    lib.check(L.kvl_mla_capture_begin(), "capture")
    rc = dec(do, dx, B, C.byref(cfg), C.byref(w), arr, lib.NO_ADVANCE)
    ge = C.c_void_p()
    lib.check(L.kvl_mla_capture_end(C.byref(ge)), "capture end")
    lib.check(rc, "captured decode")
    for r in range(3):
        zero = np.zeros_like(eager)
        lib.check(L.kvl_mla_copy_to_device(do, zero.ctypes.data, zero.nbytes), "clear")
        lib.check(L.kvl_mla_graph_launch(ge), "replay")
        lib.check(L.kvl_mla_synchronize(), "sync")
        rep = np.zeros_like(eager)
        lib.check(L.kvl_mla_copy_to_host(rep.ctypes.data, do, rep.nbytes), "d2h")
        np.testing.assert_array_equal(rep, eager, err_msg=f"replay {r}")
    lib.check(L.kvl_mla_graph_destroy(ge), "destroy")
    L.kvl_mla_device_free(dx)
    L.kvl_mla_device_free(do)
    # the host API over the same states (rows [0, len) on the device, so nothing re-uploads)
    for st in sts:
        lib.check(L.kvl_mla_compressed_bf16_state_pull(C.byref(st), 0, st.len), "pull")
    pos = np.ascontiguousarray(lens, dtype=np.int32)
    host = np.zeros_like(eager)
    lib.check(L.kvl_mla_decode_compressed_bf16_batch_bf16(f32(host), f32(xb), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                                          B, C.byref(cfg), C.byref(w), arr), "host decode")
    np.testing.assert_array_equal(host, eager)
    # rollback: truncate to the old length and decode the same token again
    again = np.zeros(H, np.float32)
    lib.check(L.kvl_mla_compressed_bf16_state_truncate(C.byref(sts[3]), lens[3]), "truncate")
    lib.check(L.kvl_mla_decode_compressed_bf16_bf16(f32(again), f32(xb[3]), lens[3], C.byref(cfg), C.byref(w),
                                                     C.byref(sts[3])), "re-decode")
    lone = np.zeros(H, np.float32)
    st = new_bf16(cfg, lens[3] + 2)
    lib.check(L.kvl_mla_compressed_bf16_state_fill_synthetic(C.byref(st), 0, lens[3], 0xB53), "fill")
    lib.check(L.kvl_mla_decode_compressed_bf16_bf16(f32(lone), f32(xb[3]), lens[3], C.byref(cfg), C.byref(w),
                                                     C.byref(st)), "lone decode")
    np.testing.assert_array_equal(again, lone)
    for s in sts + [st]:
        L.kvl_mla_compressed_bf16_state_free(C.byref(s))
    L.kvl_mla_release_weights(C.byref(w))


def test_fused_prefill_fills_the_same_rows():
    """kvl_mla_prefill_compressed_bf16_state_* (src/generate.c:208-210 as one call): state rows
    bit-identical to the state prefill's, output within the rounding of kv_a of the plain
    prefill's, the device variant equal to the host variant; then a decode continues from it."""
    cfg, layer, x = model(KIMI, 0xB6, n=300)
    w = layer.struct()
    S, H = 297, cfg.hidden_size
    xs = np.ascontiguousarray(x[:S])
    plain = np.zeros((S, H), np.float32)
    lib.check(L.kvl_mla_prefill_bf16(f32(plain), f32(xs), S, C.byref(cfg), C.byref(w)), "prefill")
    sep = new_bf16(cfg, S + 3)
    lib.check(L.kvl_mla_compressed_bf16_state_prefill_bf16(f32(xs), S, C.byref(cfg), C.byref(w), C.byref(sep)),
              "state prefill")
    fus = new_bf16(cfg, S + 3)
    out = np.zeros_like(plain)
    lib.check(L.kvl_mla_prefill_compressed_bf16_state_bf16(f32(out), f32(xs), S, C.byref(cfg), C.byref(w),
                                                           C.byref(fus)), "fused")
    assert sep.len == fus.len == S
    for a, b in zip(rows_of(fus, S), rows_of(sep, S)):
        np.testing.assert_array_equal(a, b)
    print(f"[bf16] fused vs plain prefill {rel_err(out, plain):.3e}", flush=True)
    assert rel_err(out, plain) <= 1e-4
    dev = new_bf16(cfg, S + 3)
    dx, do = L.kvl_mla_device_alloc(xs.nbytes), L.kvl_mla_device_alloc(xs.nbytes)
    lib.check(L.kvl_mla_copy_to_device(dx, xs.ctypes.data, xs.nbytes), "h2d")
    lib.check(L.kvl_mla_prefill_compressed_bf16_state_device(do, dx, S, C.byref(cfg), C.byref(w), C.byref(dev)),
              "fused device")
    od = np.zeros_like(out)
    lib.check(L.kvl_mla_copy_to_host(od.ctypes.data, do, od.nbytes), "d2h")
    lib.check(L.kvl_mla_compressed_bf16_state_pull(C.byref(dev), 0, S), "pull")
    np.testing.assert_array_equal(od, out)
    for a, b in zip(rows_of(dev, S), rows_of(fus, S)):
        np.testing.assert_array_equal(a, b)
    L.kvl_mla_device_free(dx)
    L.kvl_mla_device_free(do)
    got = np.zeros(H, np.float32)
    lib.check(L.kvl_mla_decode_compressed_bf16_bf16(f32(got), f32(x[S]), S, C.byref(cfg), C.byref(w), C.byref(fus)),
              "decode after fused prefill")
    twin = new_twin(cfg, S + 3)
    ref, _ = oracle_decode(cfg, w, twin, fus, x[S], S)
    assert rel_err(got, ref) <= TOL
    for s in (sep, fus, dev):
        L.kvl_mla_compressed_bf16_state_free(C.byref(s))
    O.mla_compressed_state_free(C.byref(twin))


def test_attention_layer_bf16():
    """kvl_mla_attention_layer_bf16_device (src/generate.c:34-67 for a batch): bit-identical to the
    same composition through the host API, and the attention increment within 2e-3 of the
    oracle's composition over the same bf16 rows."""
    cfg, layer, _ = model(KIMI, 0xB7)
    w = layer.struct()
    H = cfg.hidden_size
    rng = np.random.default_rng(0xB7)
    in_norm = inputs.f32_to_bf16_bits(1.0 + 0.02 * rng.standard_normal(H).astype(np.float32))
    post_norm = inputs.f32_to_bf16_bits(1.0 + 0.02 * rng.standard_normal(H).astype(np.float32))
    lens = [700, 1200, 333]
    B = len(lens)
    h0 = np.ascontiguousarray(inputs.hidden(cfg, 0xB8, B))

    def states():
        sts = []
        for i, n in enumerate(lens):
            st = new_bf16(cfg, n + 2)
            lib.check(L.kvl_mla_compressed_bf16_state_fill_synthetic(C.byref(st), 0, n, 0xB70 + i), "fill")
            lib.check(L.kvl_mla_compressed_bf16_state_pull(C.byref(st), 0, n), "pull")
            sts.append(st)
        return sts, (BSP * B)(*[C.pointer(s) for s in sts])

    dsts, darr = states()
    d_h, d_n2 = L.kvl_mla_device_alloc(h0.nbytes), L.kvl_mla_device_alloc(h0.nbytes)
    lib.check(L.kvl_mla_copy_to_device(d_h, h0.ctypes.data, h0.nbytes), "h2d")
    lib.check(L.kvl_mla_attention_layer_bf16_device(d_h, d_n2, B, C.byref(cfg), C.byref(w),
                                                    in_norm.ctypes.data_as(abi.u16p),
                                                    post_norm.ctypes.data_as(abi.u16p), darr, 0), "layer")
    h1, n2 = np.zeros_like(h0), np.zeros_like(h0)
    lib.check(L.kvl_mla_copy_to_host(h1.ctypes.data, d_h, h0.nbytes), "d2h")
    lib.check(L.kvl_mla_copy_to_host(n2.ctypes.data, d_n2, h0.nbytes), "d2h")
    assert [s.len for s in dsts] == [n + 1 for n in lens]
    hsts, harr = states()
    n1 = np.zeros_like(h0)
    for b in range(B):
        L.kvl_rmsnorm_bf16(f32(n1[b]), f32(h0[b]), in_norm.ctypes.data_as(abi.u16p), H, np.float32(cfg.rms_eps))
    attn = np.zeros_like(h0)
    pos = np.array(lens, np.int32)
    lib.check(L.kvl_mla_decode_compressed_bf16_batch_bf16(f32(attn), f32(n1), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                                          B, C.byref(cfg), C.byref(w), harr), "host decode")
    r1 = (h0 + attn).astype(np.float32)
    n2h = np.zeros_like(h0)
    for b in range(B):
        L.kvl_rmsnorm_bf16(f32(n2h[b]), f32(r1[b]), post_norm.ctypes.data_as(abi.u16p), H, np.float32(cfg.rms_eps))
    np.testing.assert_array_equal(h1, r1)
    np.testing.assert_array_equal(n2, n2h)
    twin = new_twin(cfg, max(lens) + 2)
    worst = 0.0
    for b in range(B):
        ref, _ = oracle_decode(cfg, w, twin, hsts[b], n1[b], lens[b])
        worst = max(worst, rel_err(h1[b] - h0[b], ref))
    print(f"[bf16] attention layer increment vs oracle {worst:.3e}", flush=True)
    assert worst <= TOL
    L.kvl_mla_device_free(d_h)
    L.kvl_mla_device_free(d_n2)
    for s in dsts + hsts:
        L.kvl_mla_compressed_bf16_state_free(C.byref(s))
    O.mla_compressed_state_free(C.byref(twin))
