"""Pins the CPU oracle (oracle/kvl_oracle.c) before anything is checked against it.

Three independent anchors:
1. the reference MLA path compiled from its own sources (oracle/_ref), compared bit for bit
   in both of its build flavours (scalar double GEMV, AVX2 8-lane FP32 GEMV);
2. closed forms and invariants (BF16 rounding, the quantizer's special cases, RoPE at
   position 0 and its pair norms, RMSNorm, a float64 textbook MLA on small shapes);
3. the reference probes' own gates (src/mla_incremental_probe.c:105,
   src/spec_q8_lab_probe.c:173-181, src/mla_streaming_probe.c:89).
"""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import Api, decode_seq, f32, i8, rel_err, u16, dequant
from kvl_mla import inputs
from kvl_mla.inputs import bf16_bits_to_f32, f32_to_bf16_bits

ORC = pyoracle.load_oracle()
O = Api(ORC, "orc_")

# small shapes of the reference probes
TINY = dict(hidden_size=16, num_heads=2, qk_nope_dim=4, qk_rope_dim=4, v_head_dim=4,
            kv_lora_rank=6, rms_eps=1e-6, rope_theta=10000.0)      # mla_incremental_probe.c:33,58
LAB = dict(hidden_size=64, num_heads=4, qk_nope_dim=8, qk_rope_dim=8, v_head_dim=8,
           kv_lora_rank=32, rms_eps=1e-6, rope_theta=10000.0)      # spec_q8_lab_probe.c:44-46,83
STREAM = dict(hidden_size=16, num_heads=2, qk_nope_dim=4, qk_rope_dim=4, v_head_dim=8,
              kv_lora_rank=6, rms_eps=1e-5, rope_theta=800000.0)   # mla_streaming_probe.c:39,46


def cfg_of(d):
    return inputs.config(**d)


def model(d, seed, std=0.2, n=8, xstd=0.25):
    cfg = cfg_of(d)
    layer = inputs.make_layer(cfg, seed, std=std)
    x = (inputs.hidden(cfg, seed, n) * np.float32(xstd)).astype(np.float32)
    return cfg, layer, x


@pytest.fixture(params=["avx2", "scalar"])
def order(request):
    ORC.orc_set_order(pyoracle.ORDER[request.param])
    yield request.param
    ORC.orc_set_order(pyoracle.ORDER["avx2"])


def ref_or_skip(kind):
    lib = pyoracle.load_reference(kind)
    if lib is None:
        pytest.skip("reference build (oracle/_ref) not present")
    return Api(lib, "kvl_")


# ---------------------------------------------------------------- closed forms --------

def test_bf16_to_f32_all_words():
    # NaN words are checked by class only: the float return through ctypes (float -> Python
    # double -> float32) quietens signalling NaN payloads.
    words = np.arange(0, 65536, 7, dtype=np.uint16)
    got = np.array([ORC.orc_bf16_to_f32(int(w)) for w in words], dtype=np.float32)
    want = (words.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(want)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))


def _bf16_nearest_even(x):
    """Independent RNE: choose the nearer of the two bracketing BF16 values in float64,
    ties to the even mantissa. Finite inputs whose rounding stays finite only."""
    u = np.float32(x).view(np.uint32)
    lo = np.uint32(u & 0xFFFF0000)
    hi = np.uint32(lo + 0x10000)
    vl = np.float64(np.uint32(lo).view(np.float32))
    vh = np.float64(np.uint32(hi).view(np.float32))
    xv = np.float64(np.float32(x))
    dl, dh = abs(xv - vl), abs(vh - xv)
    if dl < dh:
        return int(lo >> 16)
    if dh < dl:
        return int(hi >> 16)
    return int(lo >> 16) if ((lo >> 16) & 1) == 0 else int(hi >> 16)


def test_bf16_rne_matches_nearest_even():
    rng = np.random.default_rng(7)
    vals = list(rng.standard_normal(2000).astype(np.float32))
    # exact ties: low half 0x8000 with even and odd retained mantissa
    vals += [np.uint32(0x3F808000).view(np.float32), np.uint32(0x3F818000).view(np.float32),
             np.uint32(0xBF808000).view(np.float32), np.float32(1e-40), np.float32(-0.0)]
    for v in vals:
        assert ORC.orc_f32_to_bf16_rne(float(v)) == _bf16_nearest_even(v), v


def test_bf16_rne_nonfinite_truncates():
    # quiet NaNs only: a signalling NaN cannot cross the ctypes float argument unchanged
    for bits in (0x7F800000, 0xFF800000, 0x7FC00001, 0xFFC12345):
        v = np.uint32(bits).view(np.float32)
        assert ORC.orc_f32_to_bf16_rne(float(v)) == bits >> 16
    # numpy mirror agrees (used to build BF16 inputs)
    v = np.array([1.0, -2.5, 3.1415927, 1e30, -1e-30], dtype=np.float32)
    assert [ORC.orc_f32_to_bf16_rne(float(a)) for a in v] == list(f32_to_bf16_bits(v))


def quantize(x):
    codes = np.zeros(x.size, dtype=np.int8)
    scale = np.zeros(1, dtype=np.float32)
    ORC.orc_quantize_latent(i8(codes), f32(scale), f32(np.ascontiguousarray(x, np.float32)),
                            x.size)
    return codes, float(scale[0])


def test_quantizer_closed_form():
    x = inputs.normal_f32(3, "q", (512,))
    codes, scale = quantize(x)
    amax = np.max(np.abs(x))
    assert scale == np.float32(amax) / np.float32(127.0)
    k = int(np.argmax(np.abs(x)))
    assert codes[k] == (127 if x[k] > 0 else -127)
    assert np.all(np.abs(codes.astype(int)) <= 127)
    inv = np.float32(1.0) / np.float32(scale)
    prod = (x * inv).astype(np.float32)
    want = np.clip(np.sign(prod) * np.floor(np.abs(prod).astype(np.float64) + 0.5), -127, 127)
    np.testing.assert_array_equal(codes, want.astype(np.int8))
    # dequantisation error bound: |x - q*s| <= s/2 (+ rounding of the product)
    deq = codes.astype(np.float32) * np.float32(scale)
    assert np.max(np.abs(deq - x)) <= 0.5 * scale * (1 + 1e-5)


def test_quantizer_special_rows():
    for row in (np.zeros(64, np.float32), np.full(64, np.nan, np.float32),
                np.array([1.0, np.inf] + [0.0] * 62, np.float32)):
        codes, scale = quantize(row)
        assert scale == 1.0 and not codes.any()


def test_quantizer_rounds_half_away_from_zero():
    # amax = 127 -> scale 1, inv 1: x = k + 0.5 must round away from zero (roundf)
    x = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 3.5, -126.5] + [0.0] * 9, dtype=np.float32)
    codes, scale = quantize(x)
    assert scale == 1.0
    assert list(codes[:7]) == [127, 3, -3, 1, -1, 4, -127]


def rope(raw, pos, theta):
    out = np.zeros_like(raw)
    ORC.orc_rope_interleaved(f32(out), f32(raw), raw.size, pos, theta)
    return out


def test_rope_position_zero_is_even_odd_permutation():
    raw = inputs.normal_f32(1, "r", (64,))
    np.testing.assert_array_equal(rope(raw, 0, 5e4), np.concatenate([raw[0::2], raw[1::2]]))


def test_rope_preserves_pair_norms_and_matches_rotate_half():
    raw = inputs.normal_f32(2, "r", (64,))
    theta, pos = 50000.0, 12345
    got = rope(raw, pos, theta).astype(np.float64)
    half = 32
    n_in = raw[0::2].astype(np.float64) ** 2 + raw[1::2].astype(np.float64) ** 2
    n_out = got[:half] ** 2 + got[half:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5)
    # torch-style formulation of the reference's test oracle (tests/test_layer_oracle.py:17-28):
    # reshape [D/2,2] -> transpose -> flatten, then q*cos + rotate_half(q)*sin
    q = raw.astype(np.float64).reshape(half, 2).T.reshape(-1)
    inv = theta ** (-np.arange(0, 64, 2, dtype=np.float64) / 64)
    ang = np.concatenate([pos * inv, pos * inv])
    rot = np.concatenate([-q[half:], q[:half]])
    want = q * np.cos(ang) + rot * np.sin(ang)
    np.testing.assert_allclose(got, want, rtol=0, atol=3e-6 * np.max(np.abs(want)))


def test_rmsnorm_closed_form():
    x = inputs.normal_f32(4, "x", (512,)) * np.float32(3.0)
    w = inputs.normal_bf16(4, "w", (512,), mean=1.0, std=0.1)
    y = np.zeros(512, np.float32)
    ORC.orc_rmsnorm_bf16(f32(y), f32(x), u16(w), 512, np.float32(1e-5))
    ms = np.mean(x.astype(np.float64) ** 2)
    want = x.astype(np.float64) / np.sqrt(ms + 1e-5) * bf16_bits_to_f32(w)
    np.testing.assert_allclose(y, want, rtol=3e-7, atol=0)


@pytest.mark.parametrize("n", [7, 64, 2048, 2051])
def test_gemv_against_float64(order, n):
    x = inputs.normal_f32(5, "x", (n,))
    w = inputs.normal_bf16(5, "w", (96, n), std=0.02)
    y = np.zeros(96, np.float32)
    ORC.orc_matvec_bf16(f32(y), f32(x), u16(w), n, 96)
    want = bf16_bits_to_f32(w).astype(np.float64) @ x.astype(np.float64)
    tol = 1e-6 if order == "scalar" else 4e-6 * np.sqrt(n / 64)
    assert rel_err(y, want) < tol


# ------------------------------------------------- bit-exact against the reference ----

@pytest.mark.parametrize("kind", ["avx2", "scalar"])
def test_gemv_rmsnorm_bit_exact_vs_reference(kind):
    R = ref_or_skip(kind)
    ORC.orc_set_order(pyoracle.ORDER[kind])
    try:
        for n, out in ((2048, 576), (512, 256), (13, 70)):
            x = inputs.normal_f32(n, "x", (n,))
            w = inputs.normal_bf16(n, "w", (out, n), std=0.05)
            a = np.zeros(out, np.float32)
            b = np.zeros(out, np.float32)
            ORC.orc_matvec_bf16(f32(a), f32(x), u16(w), n, out)
            R.matvec_bf16(f32(b), f32(x), u16(w), n, out)
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        x = inputs.normal_f32(9, "x", (512,))
        w = inputs.normal_bf16(9, "w", (512,), mean=1.0, std=0.02)
        a = np.zeros(512, np.float32)
        b = np.zeros(512, np.float32)
        ORC.orc_rmsnorm_bf16(f32(a), f32(x), u16(w), 512, np.float32(1e-5))
        R.rmsnorm_bf16(f32(b), f32(x), u16(w), 512, np.float32(1e-5))
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        ORC.orc_set_order(1)


SHAPES = [("tiny", TINY, 0.2, 9), ("lab", LAB, 0.05, 13), ("kimi", inputs.KIMI, 0.02, 6)]


@pytest.mark.parametrize("kind", ["avx2", "scalar"])
@pytest.mark.parametrize("name,dims,std,S", SHAPES, ids=[s[0] for s in SHAPES])
def test_decode_paths_bit_exact_vs_reference(kind, name, dims, std, S):
    R = ref_or_skip(kind)
    ORC.orc_set_order(pyoracle.ORDER[kind])
    try:
        cfg, layer, x = model(dims, 11, std=std, n=S, xstd=1.0)
        w = layer.struct()
        for st in ("exp", "f32", "q8"):
            for prefix in ((0,) if st == "exp" else (0, S // 2)):
                a, sa = decode_seq(O, st, cfg, w, x, prefix=prefix)
                b, sb = decode_seq(R, st, cfg, w, x, prefix=prefix)
                np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32),
                                              err_msg=f"{st} prefix={prefix}")
                for k in sa:
                    np.testing.assert_array_equal(sa[k], sb[k], err_msg=f"{st} state {k}")
    finally:
        ORC.orc_set_order(1)


@pytest.mark.parametrize("kind", ["avx2", "scalar"])
@pytest.mark.parametrize("name,dims,std,S", [("stream", STREAM, 0.2, 64), ("lab", LAB, 0.05, 33),
                                              ("kimi", inputs.KIMI, 0.02, 5)],
                         ids=["stream", "lab", "kimi"])
def test_prefill_bit_exact_vs_reference(kind, name, dims, std, S):
    R = ref_or_skip(kind)
    ORC.orc_set_order(pyoracle.ORDER[kind])
    try:
        cfg, layer, x = model(dims, 21, std=std, n=S, xstd=0.25)
        w = layer.struct()
        H = cfg.hidden_size
        a = np.zeros((S, H), np.float32)
        b = np.zeros((S, H), np.float32)
        assert ORC.orc_mla_prefill_streaming(f32(a), f32(x), S, C.byref(cfg), C.byref(w)) == 0
        assert R.mla_prefill_bf16(f32(b), f32(x), S, C.byref(cfg), C.byref(w)) == 0
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        assert ORC.orc_mla_prefill_materialized(f32(a), f32(x), S, C.byref(cfg), C.byref(w)) == 0
        assert R.mla_prefill_materialized_bf16(f32(b), f32(x), S, C.byref(cfg),
                                               C.byref(w)) == 0
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        ORC.orc_set_order(1)


def test_state_bytes_and_errors_match_reference():
    R = ref_or_skip("avx2")
    cfg = cfg_of(LAB)
    for api in (O, R):
        q = __import__("kvl_mla.abi", fromlist=["x"]).KvlMlaCompressedQ8State()
        assert api.mla_compressed_q8_state_init(C.byref(q), C.byref(cfg), 17) == 0
        assert api.mla_compressed_q8_state_bytes(C.byref(q)) == C.sizeof(q) + 17 * (32 + 4 + 16)
        assert api.mla_compressed_q8_state_truncate(C.byref(q), 1) == -1  # beyond len
        api.mla_compressed_q8_state_free(C.byref(q))
        assert q.capacity == 0 and not q.latent_q8
    bad = cfg_of(dict(LAB, qk_rope_dim=7))
    from kvl_mla.abi import KvlMlaCompressedState
    for api in (O, R):
        assert api.mla_compressed_state_init(C.byref(KvlMlaCompressedState()), C.byref(bad),
                                             4) == -1


# ------------------------------------------- the reference probes' equivalence gates ----

def test_incremental_equivalences():
    """src/mla_incremental_probe.c:60-105: expanded decode, compressed decode and state
    prefill + decode all reproduce causal prefill rows."""
    cfg, layer, x = model(TINY, 31, std=0.1, n=5, xstd=0.5)
    w = layer.struct()
    pre = np.zeros((5, 16), np.float32)
    assert O.prefill(pre, x, 5, cfg, w) == 0
    exp, _ = decode_seq(O, "exp", cfg, w, x)
    cmp, _ = decode_seq(O, "f32", cfg, w, x)
    nxt, _ = decode_seq(O, "f32", cfg, w, x, prefix=4)
    assert np.max(np.abs(exp - pre)) <= 1e-6
    assert np.max(np.abs(cmp - pre)) <= 2e-6
    assert np.max(np.abs(nxt - pre[4:])) <= 2e-6


def test_bad_order_rejected_state_unchanged():
    cfg, layer, x = model(TINY, 32, n=3)
    w = layer.struct()
    from kvl_mla.abi import KvlMlaCompressedQ8State
    s = KvlMlaCompressedQ8State()
    assert O.mla_compressed_q8_state_init(C.byref(s), C.byref(cfg), 3) == 0
    out = np.zeros(16, np.float32)
    assert O.mla_decode_compressed_q8_bf16(f32(out), f32(x[0]), 1, C.byref(cfg), C.byref(w),
                                           C.byref(s)) == -1
    assert s.len == 0
    for t in range(3):
        assert O.mla_decode_compressed_q8_bf16(f32(out), f32(x[t]), t, C.byref(cfg),
                                               C.byref(w), C.byref(s)) == 0
    assert O.mla_decode_compressed_q8_bf16(f32(out), f32(x[0]), 3, C.byref(cfg), C.byref(w),
                                           C.byref(s)) == -1  # capacity
    O.mla_compressed_q8_state_free(C.byref(s))


def test_block_and_rollback_exact_and_q8_gate():
    """src/spec_q8_lab_probe.c:86-181 at its shapes (S=13, PREFIX=5, BLOCK=4, ACCEPT=2)."""
    from kvl_mla.abi import KvlMlaCompressedState
    cfg, layer, x = model(LAB, 41, std=0.03, n=13, xstd=0.2)
    w = layer.struct()
    H, P, B, A = 64, 5, 4, 2
    seq, _ = decode_seq(O, "f32", cfg, w, x)
    st = KvlMlaCompressedState()
    assert O.mla_compressed_state_init(C.byref(st), C.byref(cfg), 14) == 0
    assert O.mla_compressed_state_prefill_bf16(f32(x[:P]), P, C.byref(cfg), C.byref(w),
                                               C.byref(st)) == 0
    blk = np.zeros((B, H), np.float32)
    assert O.mla_decode_compressed_block_bf16(f32(blk), f32(np.ascontiguousarray(x[P:P + B])),
                                              B, P, C.byref(cfg), C.byref(w), C.byref(st)) == 0
    assert np.array_equal(blk, seq[P:P + B])
    rep = inputs.normal_f32(41, "rep", (H,)) * np.float32(0.2)
    assert O.mla_compressed_state_truncate(C.byref(st), P + A) == 0
    a = np.zeros(H, np.float32)
    assert O.mla_decode_compressed_bf16(f32(a), f32(rep), P + A, C.byref(cfg), C.byref(w),
                                        C.byref(st)) == 0
    xr = np.concatenate([x[:P + A], rep[None]]).astype(np.float32)
    fresh, _ = decode_seq(O, "f32", cfg, w, xr, prefix=P + A)
    assert np.array_equal(a, fresh[0])
    O.mla_compressed_state_free(C.byref(st))
    q8, _ = decode_seq(O, "q8", cfg, w, x, prefix=P)
    d = q8.astype(np.float64) - seq[P:].astype(np.float64)
    rel_rms = np.sqrt(np.sum(d * d) / np.sum(seq[P:].astype(np.float64) ** 2))
    assert np.max(np.abs(d)) <= 0.02 and rel_rms <= 0.02


@pytest.mark.parametrize("S", [1, 7, 64, 257])
def test_streaming_equals_materialized(S):
    """src/mla_streaming_probe.c:68-89 gate: max_abs and rel_rms <= 2e-5."""
    cfg, layer, x = model(STREAM, 50 + S, std=0.2, n=S, xstd=0.25)
    w = layer.struct()
    a = np.zeros((S, 16), np.float32)
    b = np.zeros((S, 16), np.float32)
    assert ORC.orc_mla_prefill_streaming(f32(a), f32(x), S, C.byref(cfg), C.byref(w)) == 0
    assert ORC.orc_mla_prefill_materialized(f32(b), f32(x), S, C.byref(cfg), C.byref(w)) == 0
    d = a.astype(np.float64) - b
    assert np.max(np.abs(d)) <= 2e-5
    assert np.sqrt(np.sum(d * d) / (np.sum(b.astype(np.float64) ** 2) + 1e-30)) <= 2e-5


# ------------------------------------------------ float64 textbook MLA (brute force) ----

def textbook_mla(cfg, layer, x):
    """Non-absorbed causal MLA in float64, written from the model definition, not from the
    reference loops: RoPE on interleaved pairs, softmax(QK^T/sqrt(QD)) V, o_proj."""
    H, NH = cfg.hidden_size, cfg.num_heads
    DN, DR, DV, R = cfg.qk_nope_dim, cfg.qk_rope_dim, cfg.v_head_dim, cfg.kv_lora_rank
    S = x.shape[0]
    f = lambda a: bf16_bits_to_f32(a).astype(np.float64)  # noqa: E731
    Wq, Wa, nw, Wb, Wo = (f(layer.q_proj), f(layer.kv_a_proj), f(layer.kv_a_norm),
                          f(layer.kv_b_proj), f(layer.o_proj))
    X = x.astype(np.float64)
    q = (X @ Wq.T).reshape(S, NH, DN + DR)
    ka = X @ Wa.T
    lat = ka[:, :R] / np.sqrt(np.mean(ka[:, :R] ** 2, axis=1, keepdims=True) + cfg.rms_eps) * nw
    kv = (lat @ Wb.T).reshape(S, NH, DN + DV)
    inv = cfg.rope_theta ** (-np.arange(0, DR, 2) / DR)

    def rot(v, t):  # v [..., DR] interleaved pairs -> [evens', odds']
        a, b = v[..., 0::2], v[..., 1::2]
        c, s = np.cos(t * inv), np.sin(t * inv)
        return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)

    kr = np.stack([rot(ka[t, R:], t) for t in range(S)])
    out = np.zeros((S, H))
    for t in range(S):
        heads = []
        for h in range(NH):
            qh = np.concatenate([q[t, h, :DN], rot(q[t, h, DN:], t)])
            K = np.concatenate([kv[:t + 1, h, :DN], kr[:t + 1]], axis=1)
            sc = K @ qh / np.sqrt(DN + DR)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            heads.append(p @ kv[:t + 1, h, DN:])
        out[t] = Wo @ np.concatenate(heads)
    return out


@pytest.mark.parametrize("dims,S", [(TINY, 9), (LAB, 17)], ids=["tiny", "lab"])
def test_oracle_matches_float64_textbook(dims, S):
    cfg, layer, x = model(dims, 61, std=0.1, n=S, xstd=0.5)
    w = layer.struct()
    want = textbook_mla(cfg, layer, x)
    pre = np.zeros((S, cfg.hidden_size), np.float32)
    assert O.prefill(pre, x, S, cfg, w) == 0
    assert rel_err(pre, want) < 2e-6
    dec, _ = decode_seq(O, "f32", cfg, w, x)
    assert rel_err(dec, want) < 2e-6


def test_position_zero_decode_closed_form():
    """One history row: softmax weight 1, so out = o_proj . concat_h(W_UV[h] . latent_0)."""
    cfg, layer, x = model(LAB, 71, std=0.05, n=1, xstd=1.0)
    w = layer.struct()
    out, snap = decode_seq(O, "f32", cfg, w, x)
    f = lambda a: bf16_bits_to_f32(a).astype(np.float64)  # noqa: E731
    Wb = f(layer.kv_b_proj).reshape(4, 16, 32)
    lat0 = snap["latent"][0].astype(np.float64)
    ho = np.concatenate([Wb[h, 8:] @ lat0 for h in range(4)])
    np.testing.assert_allclose(out[0], f(layer.o_proj) @ ho, rtol=0, atol=1e-6)


@pytest.mark.parametrize("name,dims,std,S,rows", [
    ("stream", STREAM, 0.2, 64, [0, 1, 31, 63]),
    ("lab", LAB, 0.05, 33, [32, 0, 17]),
    ("kimi", inputs.KIMI, 0.02, 24, [0, 5, 23])], ids=["stream", "lab", "kimi"])
def test_prefill_rows_equal_full_prefill(name, dims, std, S, rows):
    """orc_mla_prefill_streaming_rows (the checker of long GPU prefills) reproduces the listed
    rows of the full streaming prefill -- itself bit-exact with the reference build -- bit for
    bit, in any row order; rows past the sequence are rejected."""
    cfg, layer, x = model(dims, 23, std=std, n=S, xstd=0.25)
    w = layer.struct()
    H = cfg.hidden_size
    full = np.zeros((S, H), np.float32)
    assert ORC.orc_mla_prefill_streaming(f32(full), f32(x), S, C.byref(cfg), C.byref(w)) == 0
    idx = np.ascontiguousarray(rows, dtype=np.int32)
    part = np.zeros((len(rows), H), np.float32)
    ip = idx.ctypes.data_as(C.POINTER(C.c_int))
    assert ORC.orc_mla_prefill_streaming_rows(f32(part), f32(x), S, ip, len(rows), C.byref(cfg), C.byref(w)) == 0
    np.testing.assert_array_equal(part.view(np.uint32), full[idx].view(np.uint32))
    bad = np.ascontiguousarray([0, S], dtype=np.int32)
    assert ORC.orc_mla_prefill_streaming_rows(f32(part), f32(x), S, bad.ctypes.data_as(C.POINTER(C.c_int)), 2,
                                              C.byref(cfg), C.byref(w)) == -1


def absorbed_decode_f64(cfg, layer, xt, lat, rope):
    """Decode output of token xt at position len(lat) - 1 over the given history rows (lat [L, R],
    rope [L, DR], rotated keys), in float64 from the model definition: per head
    q_lat = W_UK^T q_nope, scores (q_lat . c_j + RoPE(q_rope) . k_j) / sqrt(QD), softmax,
    W_UV . sum_j p_j c_j, then o_proj."""
    NH, DN, DR, DV = cfg.num_heads, cfg.qk_nope_dim, cfg.qk_rope_dim, cfg.v_head_dim
    R = cfg.kv_lora_rank
    f = lambda a: bf16_bits_to_f32(a).astype(np.float64)  # noqa: E731
    Wq, Wb, Wo = f(layer.q_proj), f(layer.kv_b_proj).reshape(NH, DN + DV, R), f(layer.o_proj)
    t = lat.shape[0] - 1
    q = (Wq @ xt.astype(np.float64)).reshape(NH, DN + DR)
    inv = cfg.rope_theta ** (-np.arange(0, DR, 2) / DR)
    c, s = np.cos(t * inv), np.sin(t * inv)
    C64, K64 = lat.astype(np.float64), rope.astype(np.float64)
    heads = []
    for h in range(NH):
        a, b = q[h, DN::2], q[h, DN + 1::2]
        qr = np.concatenate([a * c - b * s, b * c + a * s])
        ql = Wb[h, :DN].T @ q[h, :DN]
        sc = (C64 @ ql + K64 @ qr) / np.sqrt(DN + DR)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        heads.append(Wb[h, DN:] @ (p @ C64))
    return Wo @ np.concatenate(heads)


@pytest.mark.parametrize("dims,S,P", [(TINY, 9, 4), (LAB, 17, 8), (inputs.KIMI, 12, 6)],
                         ids=["tiny", "lab", "kimi"])
def test_bf16_rows_decode_pinned(dims, S, P):
    """orc_mla_decode_compressed_bf16_rows (the checker of the library's BF16-latent state):
    its appended rows are the bf16 rounding of the FP32 decode's rows (orc_f32_to_bf16_rne, bit
    for bit), and its outputs equal the float64 absorbed decode over its own rows; the same
    float64 decode over the FP32 decode's rows reproduces the FP32 decode (bit-exact with the
    reference build), which pins the float64 restatement itself."""
    cfg, layer, x = model(dims, 83, std=0.1 if dims is not inputs.KIMI else 0.02, n=S, xstd=0.5)
    w = layer.struct()
    R, DR, H = cfg.kv_lora_rank, cfg.qk_rope_dim, cfg.hidden_size
    sts = []
    for _ in range(2):
        st = abi_state(cfg, S + 1)
        assert O.mla_compressed_state_prefill_bf16(f32(x[:P]), P, C.byref(cfg), C.byref(w), C.byref(st)) == 0
        sts.append(st)
    fp, bf = sts
    # both start from the same bf16-valued prefix
    for st in sts:
        lat = np.ctypeslib.as_array(st.latent, ((S + 1) * R,))
        rope = np.ctypeslib.as_array(st.rope, ((S + 1) * DR,))
        lat[:P * R] = bf16_bits_to_f32(f32_to_bf16_bits(lat[:P * R].copy()))
        rope[:P * DR] = bf16_bits_to_f32(f32_to_bf16_bits(rope[:P * DR].copy()))
    moved = 0
    for t in range(P, S):
        o_fp, o_bf = np.zeros(H, np.float32), np.zeros(H, np.float32)
        # the FP32 decode over the same history (its own row t stays fp32)
        assert O.mla_decode_compressed_bf16(f32(o_fp), f32(x[t]), t, C.byref(cfg), C.byref(w), C.byref(fp)) == 0
        assert ORC.orc_mla_decode_compressed_bf16_rows(f32(o_bf), f32(x[t]), t, C.byref(cfg), C.byref(w),
                                                       C.byref(bf)) == 0
        assert bf.len == t + 1
        lf = np.ctypeslib.as_array(fp.latent, ((S + 1) * R,)).reshape(S + 1, R)
        rf = np.ctypeslib.as_array(fp.rope, ((S + 1) * DR,)).reshape(S + 1, DR)
        lb = np.ctypeslib.as_array(bf.latent, ((S + 1) * R,)).reshape(S + 1, R)
        rb = np.ctypeslib.as_array(bf.rope, ((S + 1) * DR,)).reshape(S + 1, DR)
        np.testing.assert_array_equal(lb[t].view(np.uint32), (f32_to_bf16_bits(lf[t].copy()).astype(np.uint32) << 16))
        np.testing.assert_array_equal(rb[t].view(np.uint32), (f32_to_bf16_bits(rf[t].copy()).astype(np.uint32) << 16))
        assert rel_err(o_fp, absorbed_decode_f64(cfg, layer, x[t], lf[:t + 1], rf[:t + 1])) < 2e-6
        assert rel_err(o_bf, absorbed_decode_f64(cfg, layer, x[t], lb[:t + 1], rb[:t + 1])) < 2e-6
        moved += int(np.any(o_bf != o_fp))
        # continue both from the bf16 row, so the next step again shares its history
        lf[t], rf[t] = lb[t], rb[t]
    assert moved > 0  # the rounding of the appended row is visible in the outputs
    for st in sts:
        O.mla_compressed_state_free(C.byref(st))


def abi_state(cfg, cap):
    from kvl_mla import abi
    st = abi.KvlMlaCompressedState()
    assert O.mla_compressed_state_init(C.byref(st), C.byref(cfg), cap) == 0
    return st
