"""Parity of the MI355X library (C ABI) with the oracle on the decode path.

Bars: quantiser-boundary rows (codes, scale, BF16 RoPE) and RMSNorm bit-exact; attention
outputs max|got - ref| / max|ref| <= 2e-3. Shapes: the reference probes' small shapes (generic
kernels) and the Kimi-VL shapes (MFMA kernels).
"""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import Api, decode_seq, f32, i8, rel_err, snapshot, u16
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

TOL = 2e-3
ORC = pyoracle.load_oracle()
O = Api(ORC, "orc_")
L = lib.load()
G = Api(L, "kvl_")

TINY = dict(hidden_size=16, num_heads=2, qk_nope_dim=4, qk_rope_dim=4, v_head_dim=4,
            kv_lora_rank=6, rms_eps=1e-6, rope_theta=10000.0)
LAB = dict(hidden_size=64, num_heads=4, qk_nope_dim=8, qk_rope_dim=8, v_head_dim=8,
           kv_lora_rank=32, rms_eps=1e-6, rope_theta=10000.0)
KIMI = dict(inputs.KIMI)


def model(d, seed, std=0.02, n=8, xstd=1.0, q_std=None):
    cfg = inputs.config(**d)
    layer = inputs.make_layer(cfg, seed, std=std, q_std=q_std)
    x = (inputs.hidden(cfg, seed, n) * np.float32(xstd)).astype(np.float32)
    return cfg, layer, x


def rand_rows(seed, n, R, DR, scale=1.0):
    lat = inputs.normal_f32(seed, "lat", (n, R)) * np.float32(scale)
    rope = inputs.normal_f32(seed, "rope", (n, DR))
    return np.ascontiguousarray(lat), np.ascontiguousarray(rope)


# ------------------------------------------------------------------ numeric helpers ----

def test_matvec_against_oracle():
    for n, out in ((2048, 576), (512, 4096), (13, 70), (2048, 2048)):
        x = inputs.normal_f32(n, "x", (n,))
        w = inputs.normal_bf16(n, "w", (out, n), std=0.02)
        a = np.zeros(out, np.float32)
        b = np.zeros(out, np.float32)
        L.kvl_matvec_bf16(f32(a), f32(x), u16(w), n, out)
        assert lib.last_error() == ""
        ORC.orc_matvec_bf16(f32(b), f32(x), u16(w), n, out)
        assert rel_err(a, b) < 1e-5, (n, out, rel_err(a, b))


def test_rmsnorm_bit_exact():
    for n in (512, 2048, 6):
        for seed in range(24):
            x = inputs.normal_f32(seed, "x", (n,)) * np.float32(0.1 + seed)
            w = inputs.normal_bf16(seed, "w", (n,), mean=1.0, std=0.1)
            a = np.zeros(n, np.float32)
            b = np.zeros(n, np.float32)
            L.kvl_rmsnorm_bf16(f32(a), f32(x), u16(w), n, np.float32(1e-5))
            ORC.orc_rmsnorm_bf16(f32(b), f32(x), u16(w), n, np.float32(1e-5))
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"n={n} seed={seed}")


def pack_gpu(lat, rope, pos, theta):
    n, R = lat.shape
    DR = rope.shape[1]
    codes = np.zeros((n, R), np.int8)
    scl = np.zeros(n, np.float32)
    rb = np.zeros((n, DR), np.uint16)
    posa = np.ascontiguousarray(pos, dtype=np.int32)
    rc = L.kvl_mla_q8_pack_rows(i8(codes), f32(scl), u16(rb), f32(lat), f32(rope),
                                posa.ctypes.data_as(C.POINTER(C.c_int)), n, R, DR, np.float32(theta))
    lib.check(rc, "q8_pack_rows")
    return codes, scl, rb


def pack_oracle(lat, rope, pos, theta):
    n, R = lat.shape
    DR = rope.shape[1]
    codes = np.zeros((n, R), np.int8)
    scl = np.zeros(n, np.float32)
    rb = np.zeros((n, DR), np.uint16)
    for i in range(n):
        ORC.orc_q8_pack_row(i8(codes[i]), f32(scl[i:i + 1]), u16(rb[i]), f32(lat[i]), f32(rope[i]),
                            R, DR, int(pos[i]), np.float32(theta))
    return codes, scl, rb


def test_q8_rows_bit_exact_at_quantiser_boundary():
    """Codes, scales and BF16 RoPE keys equal the oracle's for the same fp32 latent
    (src/mla_compressed_q8_state.c:34-55,121-125), including the special rows."""
    n, R, DR = 1500, 512, 64
    lat, rope = rand_rows(7, n, R, DR)
    lat[:500] *= np.float32(1e-3)
    lat[500:700] *= np.float32(1e4)
    lat[3] = 0.0                                   # zero row -> scale 1, zero codes
    lat[4, 17] = np.inf                            # non-finite absmax -> zero row
    lat[5] = np.float32(1e-39)                     # subnormal row
    lat[6, :] = np.float32(127.0)
    lat[6, 1:20] = np.arange(19, dtype=np.float32) + np.float32(0.5)  # exact .5 ties
    pos = (np.arange(n) * 37) % 40000
    a = pack_gpu(lat, rope, pos, 50000.0)
    b = pack_oracle(lat, rope, pos, 50000.0)
    for x, y, name in zip(a, b, ("codes", "scale", "rope")):
        np.testing.assert_array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8), err_msg=name)


# ------------------------------------------------------------------ decode parity ------

def compare_states(kind, sa, sb, exact=False):
    if kind == "q8":
        if exact:
            for k in sa:
                np.testing.assert_array_equal(sa[k], sb[k], err_msg=k)
            return
        d = np.abs(sa["codes"].astype(int) - sb["codes"].astype(int))
        assert d.max() <= 1 and d.mean() < 0.01, (d.max(), d.mean())
        np.testing.assert_allclose(sa["scale"], sb["scale"], rtol=1e-5)
        ra, rb = inputs.bf16_bits_to_f32(sa["rope"]), inputs.bf16_bits_to_f32(sb["rope"])
        assert rel_err(ra, rb) < 1e-2
    else:
        for k in sa:
            assert rel_err(sa[k], sb[k]) < 1e-4, k


SHAPES = [("tiny", TINY, 0.2, 9), ("lab", LAB, 0.05, 13), ("kimi", KIMI, 0.02, 40)]


@pytest.mark.parametrize("name,dims,std,S", SHAPES, ids=[s[0] for s in SHAPES])
@pytest.mark.parametrize("kind", ["exp", "f32", "q8"])
def test_decode_sequence_matches_oracle(name, dims, std, S, kind):
    print(f"[decode] shape={name} kind={kind} S={S}", flush=True)
    cfg, layer, x = model(dims, 11, std=std, n=S)
    w = layer.struct()
    for prefix in ((0,) if kind == "exp" else (0, S // 2)):
        a, sa = decode_seq(G, kind, cfg, w, x, prefix=prefix)
        b, sb = decode_seq(O, kind, cfg, w, x, prefix=prefix)
        assert rel_err(a, b) <= TOL, (prefix, rel_err(a, b))
        compare_states(kind, sa, sb)


@pytest.mark.parametrize("kind", ["exp", "f32", "q8"])
def test_decode_sharp_attention(kind):
    """Large attention logits (q_proj std 8x the other weights): pins the precision of the
    score products, whose rounding the logit size amplifies."""
    print(f"[decode] kimi sharp kind={kind}", flush=True)
    cfg, layer, x = model(KIMI, 13, n=48, q_std=0.16)
    w = layer.struct()
    prefix = 0 if kind == "exp" else 24
    a, sa = decode_seq(G, kind, cfg, w, x, prefix=prefix)
    b, sb = decode_seq(O, kind, cfg, w, x, prefix=prefix)
    print(f"[decode]   max|d|/max|ref| = {rel_err(a, b):.3e}", flush=True)
    assert rel_err(a, b) <= TOL, rel_err(a, b)
    compare_states(kind, sa, sb)


def test_q8_decode_sharp_8192():
    """Large logits over a long Q8 history (split-K partials with widely different maxima)."""
    cfg, layer, _ = model(KIMI, 0xC5, q_std=0.16)
    w = layer.struct()
    n = 8192
    lat, rope = rand_rows(0xC5, n, 512, 64)
    x = inputs.hidden(cfg, 0xC5, 1, tag="query")[0]
    outs = []
    for api in (G, O):
        st = fill_q8_state(api, cfg, lat, rope, n + 1)
        out = np.zeros(cfg.hidden_size, np.float32)
        assert api.mla_decode_compressed_q8_bf16(f32(out), f32(x), n, C.byref(cfg), C.byref(w), C.byref(st)) == 0
        outs.append(out)
        api.mla_compressed_q8_state_free(C.byref(st))
    print(f"[decode]   max|d|/max|ref| = {rel_err(outs[0], outs[1]):.3e}", flush=True)
    assert rel_err(outs[0], outs[1]) <= TOL, rel_err(outs[0], outs[1])


def test_errors_leave_state_unchanged():
    cfg, layer, x = model(LAB, 5, n=3)
    w = layer.struct()
    s = abi.KvlMlaCompressedQ8State()
    assert G.mla_compressed_q8_state_init(C.byref(s), C.byref(cfg), 2) == 0
    out = np.zeros(cfg.hidden_size, np.float32)
    assert G.mla_decode_compressed_q8_bf16(f32(out), f32(x[0]), 1, C.byref(cfg), C.byref(w), C.byref(s)) == -1
    assert s.len == 0
    for t in range(2):
        assert G.mla_decode_compressed_q8_bf16(f32(out), f32(x[t]), t, C.byref(cfg), C.byref(w), C.byref(s)) == 0
    assert G.mla_decode_compressed_q8_bf16(f32(out), f32(x[2]), 2, C.byref(cfg), C.byref(w), C.byref(s)) == -1
    assert s.len == 2
    bad = inputs.config(**dict(LAB, qk_rope_dim=7))
    assert G.mla_decode_compressed_q8_bf16(f32(out), f32(x[0]), 2, C.byref(bad), C.byref(w), C.byref(s)) == -1
    G.mla_compressed_q8_state_free(C.byref(s))
    assert s.capacity == 0


@pytest.mark.parametrize("bound", [False, True], ids=["unbound", "bound"])
def test_kv_b_rewritten_in_place_refreshes_device_copies(bound):
    """Weights are cached on the device by host address. Rewriting the kv_b array in place (same
    address, new contents) must refresh its bf16 copy and the W_UK^T copy derived from it (the
    query preparation's operand at the Kimi shapes): unbound weights through the sampled digest,
    bound weights through release + bind."""
    cfg, layer, x = model(KIMI, 0xD3, n=6)
    w = layer.struct()
    old = layer.kv_b_proj.copy()
    new = inputs.normal_bf16(0xD4, "kv_b", old.shape, std=0.02)
    print(f"[decode] kv_b rewrite bound={bound}", flush=True)
    for kind in ("f32", "q8"):
        layer.kv_b_proj[...] = old
        if bound:
            lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
        a0, _ = decode_seq(G, kind, cfg, w, x, prefix=3)
        if bound:
            L.kvl_mla_release_weights(C.byref(w))
        layer.kv_b_proj[...] = new
        if bound:
            lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
        a1, _ = decode_seq(G, kind, cfg, w, x, prefix=3)
        if bound:
            L.kvl_mla_release_weights(C.byref(w))
        b1, _ = decode_seq(O, kind, cfg, w, x, prefix=3)
        print(f"[decode]   {kind}: max|d|/max|ref| = {rel_err(a1, b1):.3e}", flush=True)
        assert rel_err(a1, b1) <= TOL, (kind, rel_err(a1, b1))
        assert rel_err(a0, b1) > 10 * TOL, (kind, "stale kv_b copy")


def test_unbound_kv_b_reloaded_between_queued_device_calls():
    """Stream-ordered calls return before their kernels run. Rewriting an unbound kv_b array in
    place and calling again must not let the re-upload overtake kernels of earlier calls that
    still read the old copy: calls queued with the old kv_b (no synchronisation in between) give
    the old-weight result, the call after the rewrite the new-weight result."""
    cfg, layer, _ = model(KIMI, 0xD5)
    w = layer.struct()
    old = layer.kv_b_proj.copy()
    new = inputs.normal_bf16(0xD6, "kv_b", old.shape, std=0.02)
    B, n = 8, 16384
    states = []
    for i in range(B):
        st = abi.KvlMlaCompressedQ8State()
        assert G.mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), n + 8) == 0
        lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, n, 91 + i), "fill")
        states.append(st)
    arr = (C.POINTER(abi.KvlMlaCompressedQ8State) * B)(*[C.pointer(s) for s in states])
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xD5, B, tag="q"))
    nbytes = xb.nbytes
    dx, da, db = (L.kvl_mla_device_alloc(nbytes) for _ in range(3))
    assert dx and da and db
    lib.check(L.kvl_mla_copy_to_device(dx, xb.ctypes.data, nbytes), "h2d")

    def run(dout):
        lib.check(L.kvl_mla_decode_compressed_q8_batch_device(dout, dx, B, C.byref(cfg), C.byref(w), arr,
                                                              lib.NO_ADVANCE), "device decode")

    def fetch(dout):
        got = np.zeros_like(xb)
        lib.check(L.kvl_mla_copy_to_host(got.ctypes.data, dout, nbytes), "d2h")
        return got

    print("[decode] unbound kv_b reload between queued device calls", flush=True)
    run(da)  # reference results, synchronised
    lib.check(L.kvl_mla_synchronize(), "sync")
    ref_old = fetch(da)
    layer.kv_b_proj[...] = new
    run(db)
    lib.check(L.kvl_mla_synchronize(), "sync")
    ref_new = fetch(db)
    assert rel_err(ref_old, ref_new) > 10 * TOL
    layer.kv_b_proj[...] = old
    run(da)
    lib.check(L.kvl_mla_synchronize(), "sync")
    for _ in range(40):  # keep the stream busy with old-weight calls (a few ms of kernels)
        run(da)
    layer.kv_b_proj[...] = new  # rewrite in place while they run
    run(db)
    lib.check(L.kvl_mla_synchronize(), "sync")
    np.testing.assert_array_equal(fetch(da), ref_old, err_msg="queued old-weight calls saw the new kv_b")
    np.testing.assert_array_equal(fetch(db), ref_new)
    for p in (dx, da, db):
        L.kvl_mla_device_free(p)
    for st in states:
        G.mla_compressed_q8_state_free(C.byref(st))


@pytest.mark.parametrize("dims", [LAB, KIMI], ids=["lab", "kimi"])
def test_block_equals_serial_and_rollback_exact(dims):
    """src/spec_q8_lab_probe.c:86-173 on the GPU: block decode == per-token decode exactly;
    truncate + re-decode == fresh state prefill + decode exactly."""
    cfg, layer, x = model(dims, 41, std=0.03 if dims is LAB else 0.02, n=13, xstd=0.2)
    w = layer.struct()
    H, P, B, A = cfg.hidden_size, 5, 4, 2
    seq, _ = decode_seq(G, "f32", cfg, w, x, prefix=P)
    st = abi.KvlMlaCompressedState()
    assert G.mla_compressed_state_init(C.byref(st), C.byref(cfg), 14) == 0
    assert G.mla_compressed_state_prefill_bf16(f32(x[:P]), P, C.byref(cfg), C.byref(w), C.byref(st)) == 0
    blk = np.zeros((B, H), np.float32)
    assert G.mla_decode_compressed_block_bf16(f32(blk), f32(np.ascontiguousarray(x[P:P + B])), B, P,
                                              C.byref(cfg), C.byref(w), C.byref(st)) == 0
    np.testing.assert_array_equal(blk, seq[:B])
    rep = inputs.normal_f32(41, "rep", (H,)) * np.float32(0.2)
    assert G.mla_compressed_state_truncate(C.byref(st), P + A) == 0
    a = np.zeros(H, np.float32)
    assert G.mla_decode_compressed_bf16(f32(a), f32(rep), P + A, C.byref(cfg), C.byref(w), C.byref(st)) == 0
    xr = np.concatenate([x[:P + A], rep[None]]).astype(np.float32)
    fresh, _ = decode_seq(G, "f32", cfg, w, xr, prefix=P + A)
    np.testing.assert_array_equal(a, fresh[0])
    G.mla_compressed_state_free(C.byref(st))
    # the same for the Q8 state
    q = abi.KvlMlaCompressedQ8State()
    assert G.mla_compressed_q8_state_init(C.byref(q), C.byref(cfg), 14) == 0
    assert G.mla_compressed_q8_state_prefill_bf16(f32(x[:P + B]), P + B, C.byref(cfg), C.byref(w), C.byref(q)) == 0
    assert G.mla_compressed_q8_state_truncate(C.byref(q), P + A) == 0
    assert G.mla_decode_compressed_q8_bf16(f32(a), f32(rep), P + A, C.byref(cfg), C.byref(w), C.byref(q)) == 0
    fresh, _ = decode_seq(G, "q8", cfg, w, xr, prefix=P + A)
    np.testing.assert_array_equal(a, fresh[0])
    G.mla_compressed_q8_state_free(C.byref(q))
    # Q8 vs FP32 gate of the reference probe (src/spec_q8_lab_probe.c:177)
    q8, _ = decode_seq(G, "q8", cfg, w, x, prefix=P)
    d = q8.astype(np.float64) - seq.astype(np.float64)
    assert np.max(np.abs(d)) <= 0.02
    assert np.sqrt(np.sum(d * d) / np.sum(seq.astype(np.float64) ** 2)) <= 0.02


def fill_q8_state(api, cfg, lat, rope_raw, cap):
    """History rows written straight into the Q8 struct (as src/self_spec_sweep.c:115-134):
    reference quantiser on the fp32 latents, RoPE at the row position, BF16."""
    n, R = lat.shape
    st = abi.KvlMlaCompressedQ8State()
    assert api.mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), cap) == 0
    codes, scl, rb = pack_oracle(lat, rope_raw, np.arange(n), cfg.rope_theta)
    np.ctypeslib.as_array(st.latent_q8, (cap * R,))[:n * R] = codes.ravel()
    np.ctypeslib.as_array(st.latent_scale, (cap,))[:n] = scl
    np.ctypeslib.as_array(st.rope_bf16, (cap * cfg.qk_rope_dim,))[:n * cfg.qk_rope_dim] = rb.ravel()
    st.len = n
    return st


def test_config1_q8_decode_8192():
    """Batch 1 over an 8192-token Q8 history of N(0,1) latents quantised by absmax/127."""
    cfg, layer, _ = model(KIMI, 0xC1)
    w = layer.struct()
    n = 8192
    lat, rope = rand_rows(0xC1, n, 512, 64)
    x = inputs.hidden(cfg, 0xC1, 1, tag="query")[0]
    outs, snaps = [], []
    for api in (G, O):
        st = fill_q8_state(api, cfg, lat, rope, n + 1)
        out = np.zeros(cfg.hidden_size, np.float32)
        assert api.mla_decode_compressed_q8_bf16(f32(out), f32(x), n, C.byref(cfg), C.byref(w), C.byref(st)) == 0
        outs.append(out)
        snaps.append(snapshot("q8", st, cfg))
        api.mla_compressed_q8_state_free(C.byref(st))
    assert rel_err(outs[0], outs[1]) <= TOL, rel_err(outs[0], outs[1])
    for k in ("codes", "scale", "rope"):  # untouched history rows stay identical
        np.testing.assert_array_equal(snaps[0][k][:n], snaps[1][k][:n])
    compare_states("q8", {k: v[n:] for k, v in snaps[0].items()}, {k: v[n:] for k, v in snaps[1].items()})


def test_config0_f32_decode_1024():
    """Batch 1, FP32 history of 1024 tokens filled by the state prefill, decode token 1024."""
    cfg, layer, x = model(KIMI, 0xC0, n=1025)
    w = layer.struct()
    a, sa = decode_seq(G, "f32", cfg, w, x, prefix=1024)
    b, sb = decode_seq(O, "f32", cfg, w, x, prefix=1024)
    assert rel_err(a, b) <= TOL, rel_err(a, b)
    compare_states("f32", sa, sb)


@pytest.mark.parametrize("kind", ["f32", "q8"])
def test_batched_ragged_decode(kind):
    """Ragged batch (one query each) through the batched entry point == per-sequence oracle."""
    cfg, layer, _ = model(KIMI, 0xC2)
    w = layer.struct()
    rng = np.random.default_rng(0xC2)
    lens = rng.integers(64, 2500, size=11)
    R, DR = 512, 64
    states_g, states_o, outs_o = [], [], []
    xb = inputs.hidden(cfg, 0xC2, len(lens), tag="query")
    for i, Lb in enumerate(lens):
        lat, rope = rand_rows(1000 + i, int(Lb), R, DR)
        lat = inputs.bf16_bits_to_f32(inputs.f32_to_bf16_bits(lat))
        pair = []
        for api in (G, O):
            if kind == "q8":
                st = fill_q8_state(api, cfg, lat, rope, int(Lb) + 1)
            else:
                st = abi.KvlMlaCompressedState()
                assert api.mla_compressed_state_init(C.byref(st), C.byref(cfg), int(Lb) + 1) == 0
                np.ctypeslib.as_array(st.latent, ((int(Lb) + 1) * R,))[:Lb * R] = lat.ravel()
                rr = inputs.bf16_bits_to_f32(inputs.f32_to_bf16_bits(rope))
                np.ctypeslib.as_array(st.rope, ((int(Lb) + 1) * DR,))[:Lb * DR] = rr.ravel()
                st.len = int(Lb)
            pair.append(st)
        states_g.append(pair[0])
        states_o.append(pair[1])
    for i, st in enumerate(states_o):
        out = np.zeros(cfg.hidden_size, np.float32)
        fn = O.mla_decode_compressed_q8_bf16 if kind == "q8" else O.mla_decode_compressed_bf16
        assert fn(f32(out), f32(xb[i]), int(lens[i]), C.byref(cfg), C.byref(w), C.byref(st)) == 0
        outs_o.append(out)
    T = abi.KvlMlaCompressedQ8State if kind == "q8" else abi.KvlMlaCompressedState
    arr = (C.POINTER(T) * len(lens))(*[C.pointer(s) for s in states_g])
    pos = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.zeros((len(lens), cfg.hidden_size), np.float32)
    fn = L.kvl_mla_decode_compressed_q8_batch_bf16 if kind == "q8" else L.kvl_mla_decode_compressed_batch_bf16
    lib.check(fn(f32(out), f32(np.ascontiguousarray(xb)), pos.ctypes.data_as(C.POINTER(C.c_int)), len(lens),
                 C.byref(cfg), C.byref(w), arr), "batched decode")
    for i in range(len(lens)):
        assert rel_err(out[i], outs_o[i]) <= TOL, (i, int(lens[i]), rel_err(out[i], outs_o[i]))
        assert states_g[i].len == lens[i] + 1
    free = O.mla_compressed_q8_state_free if kind == "q8" else O.mla_compressed_state_free
    for s in states_o:
        free(C.byref(s))
    freeg = G.mla_compressed_q8_state_free if kind == "q8" else G.mla_compressed_state_free
    for s in states_g:
        freeg(C.byref(s))


def test_config2_ragged_64_sequences_bf16_cache():
    """64 sequences, context lengths uniform in [512, 32768] (seeded), each with its own
    bf16-representable latent cache (FP32 state, device-generated), one query each, through
    the batched entry point. Every sequence against a lone GPU decode of the same token (the
    batch only changes the split boundaries), and 6 of them (shortest, longest, 4 others)
    against the oracle on the pulled rows."""
    cfg, layer, _ = model(KIMI, 0xC8)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    rng = np.random.default_rng(0xC8)
    lens = rng.integers(512, 32769, size=64)
    B, H = len(lens), cfg.hidden_size
    print(f"[config2] 64 sequences, {int(lens.sum())} rows", flush=True)
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xC8, B, tag="query"))

    def make_states():
        sts = []
        for i, n in enumerate(lens):
            st = abi.KvlMlaCompressedState()
            assert G.mla_compressed_state_init(C.byref(st), C.byref(cfg), int(n) + 1) == 0
            lib.check(L.kvl_mla_compressed_state_fill_synthetic(C.byref(st), 0, int(n), 0xC80 + i), "fill")
            sts.append(st)
        return sts

    batch_states = make_states()
    arr = (C.POINTER(abi.KvlMlaCompressedState) * B)(*[C.pointer(s) for s in batch_states])
    pos = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.zeros((B, H), np.float32)
    lib.check(L.kvl_mla_decode_compressed_batch_bf16(f32(out), f32(xb), pos.ctypes.data_as(C.POINTER(C.c_int)), B,
                                                     C.byref(cfg), C.byref(w), arr), "batched decode")
    assert all(s.len == n + 1 for s, n in zip(batch_states, lens))
    for s in batch_states:
        G.mla_compressed_state_free(C.byref(s))
    print("[config2]   batch done; lone decodes", flush=True)
    lone_states = make_states()
    lone = np.zeros_like(out)
    for i, st in enumerate(lone_states):
        lib.check(L.kvl_mla_decode_compressed_bf16(f32(lone[i]), f32(xb[i]), int(lens[i]), C.byref(cfg), C.byref(w),
                                                   C.byref(st)), f"lone decode {i}")
    worst = max(rel_err(out[i], lone[i]) for i in range(B))
    print(f"[config2]   batch vs lone max rel err {worst:.3e}", flush=True)
    assert worst <= 1e-4
    picks = sorted({int(np.argmin(lens)), int(np.argmax(lens)), 5, 17, 33, 50})
    for i in picks:
        st = lone_states[i]
        n = int(lens[i])
        lib.check(L.kvl_mla_compressed_state_pull(C.byref(st), 0, n), "pull")
        st.len = n  # the oracle appends the same token at position n
        ref = np.zeros(H, np.float32)
        assert O.mla_decode_compressed_bf16(f32(ref), f32(xb[i]), n, C.byref(cfg), C.byref(w), C.byref(st)) == 0
        e = rel_err(out[i], ref)
        print(f"[config2]   sequence {i} ({n} rows) vs oracle {e:.3e}", flush=True)
        assert e <= TOL, (i, n, e)
    for s in lone_states:
        G.mla_compressed_state_free(C.byref(s))
    L.kvl_mla_release_weights(C.byref(w))


def test_synthetic_history_matches_host_mirror():
    cfg = inputs.config(**KIMI)
    st = abi.KvlMlaCompressedQ8State()
    assert G.mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), 3000) == 0
    lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, 2999, 0xC4), "fill")
    assert st.len == 2999
    lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, 2999), "pull")
    snap = snapshot("q8", st, cfg)
    rows = np.array([0, 1, 2, 777, 1500, 2998])
    lat, rope = inputs.synth_rows(0xC4, rows, 512, 64)
    for i, r in enumerate(rows):
        codes = np.zeros(512, np.int8)
        scl = np.zeros(1, np.float32)
        ORC.orc_quantize_latent(i8(codes), f32(scl), f32(np.ascontiguousarray(lat[i])), 512)
        np.testing.assert_array_equal(snap["codes"][r], codes)
        assert snap["scale"][r] == scl[0]
        np.testing.assert_array_equal(snap["rope"][r], inputs.f32_to_bf16_bits(rope[i]))
    G.mla_compressed_q8_state_free(C.byref(st))


def test_device_api_and_graph_replay_match_host_api():
    """Stream-ordered decode (device buffers, no advance) and its HIP-graph replays equal the
    synchronous host API for the same inputs, replay after replay."""
    cfg, layer, _ = model(KIMI, 0xD1)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    B, n = 4, 700
    states = []
    for i in range(B):
        st = abi.KvlMlaCompressedQ8State()
        assert G.mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), n + 8) == 0
        lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, n - 50 * i, 77 + i), "fill")
        states.append(st)
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xD1, B, tag="q"))
    arr = (C.POINTER(abi.KvlMlaCompressedQ8State) * B)(*[C.pointer(s) for s in states])
    nbytes = xb.nbytes
    dx = L.kvl_mla_device_alloc(nbytes)
    dout = L.kvl_mla_device_alloc(nbytes)
    assert dx and dout
    lib.check(L.kvl_mla_copy_to_device(dx, xb.ctypes.data, nbytes), "h2d")
    lib.check(L.kvl_mla_decode_compressed_q8_batch_device(dout, dx, B, C.byref(cfg), C.byref(w), arr,
                                                          lib.NO_ADVANCE), "device decode")
    eager = np.zeros_like(xb)
    lib.check(L.kvl_mla_copy_to_host(eager.ctypes.data, dout, nbytes), "d2h")
    assert [s.len for s in states] == [n - 50 * i for i in range(B)]
    # graph capture of the same call, replayed three times with eager work in between
    lib.check(L.kvl_mla_capture_begin(), "capture begin")
    rc = L.kvl_mla_decode_compressed_q8_batch_device(dout, dx, B, C.byref(cfg), C.byref(w), arr, lib.NO_ADVANCE)
    ge = C.c_void_p()
    lib.check(L.kvl_mla_capture_end(C.byref(ge)), "capture end")
    lib.check(rc, "captured decode")
    for rep in range(3):
        junk = np.zeros_like(xb)
        lib.check(L.kvl_mla_copy_to_device(dout, junk.ctypes.data, nbytes), "clear")
        lib.check(L.kvl_mla_graph_launch(ge), "graph launch")
        lib.check(L.kvl_mla_synchronize(), "sync")
        got = np.zeros_like(xb)
        lib.check(L.kvl_mla_copy_to_host(got.ctypes.data, dout, nbytes), "d2h")
        np.testing.assert_array_equal(got, eager, err_msg=f"replay {rep}")
        lib.check(L.kvl_mla_decode_compressed_q8_batch_device(dout, dx, B, C.byref(cfg), C.byref(w), arr,
                                                              lib.NO_ADVANCE), "eager between replays")
        lib.check(L.kvl_mla_synchronize(), "sync")
    lib.check(L.kvl_mla_graph_destroy(ge), "graph destroy")
    # host API on pulled rows gives the same numbers
    host = np.zeros_like(xb)
    for i, st in enumerate(states):
        lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, st.len), "pull")
    pos = np.array([s.len for s in states], dtype=np.int32)
    lib.check(L.kvl_mla_decode_compressed_q8_batch_bf16(f32(host), f32(xb), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                                        B, C.byref(cfg), C.byref(w), arr), "host decode")
    np.testing.assert_array_equal(host, eager)
    L.kvl_mla_device_free(dx)
    L.kvl_mla_device_free(dout)
    for st in states:
        G.mla_compressed_q8_state_free(C.byref(st))
    L.kvl_mla_release_weights(C.byref(w))


def test_stage_events_inside_a_graph():
    """Timing mode 2 records the stage events into a captured graph: after replays, every
    stage of the decode has one positive duration per launch, the graph's output equals the
    eager call's, and the durations add up to less than the replay's own time."""
    cfg, layer, _ = model(KIMI, 0xD3)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    B, n = 2, 3000
    states = []
    for i in range(B):
        st = abi.KvlMlaCompressedQ8State()
        assert G.mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), n + 4) == 0
        lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, n, 90 + i), "fill")
        states.append(st)
    xb = np.ascontiguousarray(inputs.hidden(cfg, 0xD3, B, tag="q"))
    arr = (C.POINTER(abi.KvlMlaCompressedQ8State) * B)(*[C.pointer(s) for s in states])
    nbytes = xb.nbytes
    dx, dout = L.kvl_mla_device_alloc(nbytes), L.kvl_mla_device_alloc(nbytes)
    assert dx and dout
    lib.check(L.kvl_mla_copy_to_device(dx, xb.ctypes.data, nbytes), "h2d")
    lib.check(L.kvl_mla_decode_compressed_q8_batch_device(dout, dx, B, C.byref(cfg), C.byref(w), arr,
                                                          lib.NO_ADVANCE), "eager decode")
    eager = np.zeros_like(xb)
    lib.check(L.kvl_mla_copy_to_host(eager.ctypes.data, dout, nbytes), "d2h")
    ms, cnt = (C.c_double * 6)(), (C.c_int * 6)()
    lib.check(L.kvl_mla_timing_read(ms, cnt), "clear records")
    lib.check(L.kvl_mla_timing_enable(2), "timing mode 2")
    lib.check(L.kvl_mla_capture_begin(), "capture begin")
    rc = L.kvl_mla_decode_compressed_q8_batch_device(dout, dx, B, C.byref(cfg), C.byref(w), arr, lib.NO_ADVANCE)
    ge = C.c_void_p()
    lib.check(L.kvl_mla_capture_end(C.byref(ge)), "capture end")
    lib.check(L.kvl_mla_timing_enable(0), "timing off")
    lib.check(rc, "captured decode")
    for _ in range(3):
        lib.check(L.kvl_mla_graph_launch(ge), "graph launch")
    e0 = L.kvl_mla_event_record()
    lib.check(L.kvl_mla_graph_launch(ge), "graph launch")
    e1 = L.kvl_mla_event_record()
    lib.check(L.kvl_mla_synchronize(), "sync")
    replay_ms = L.kvl_mla_event_elapsed_ms(e0, e1)
    L.kvl_mla_event_destroy(e0)
    L.kvl_mla_event_destroy(e1)
    lib.check(L.kvl_mla_timing_read(ms, cnt), "timing read")
    lib.check(L.kvl_mla_graph_destroy(ge), "graph destroy")
    got = np.zeros_like(xb)
    lib.check(L.kvl_mla_copy_to_host(got.ctypes.data, dout, nbytes), "d2h")
    np.testing.assert_array_equal(got, eager)
    stages = {name: (ms[i], cnt[i]) for i, name in enumerate(lib.STAGES)}
    print(f"[timing] graph replay {replay_ms:.4f} ms, stages {stages}", flush=True)
    for name in ("gemv_in", "append_qprep", "attention", "combine", "gemv_out"):
        t, c = stages[name]
        assert c == 1 and t > 0.0, (name, t, c)
    assert sum(t for t, _ in stages.values()) <= replay_ms * 1.001
    L.kvl_mla_device_free(dx)
    L.kvl_mla_device_free(dout)
    for st in states:
        G.mla_compressed_q8_state_free(C.byref(st))
    L.kvl_mla_release_weights(C.byref(w))
