"""Q8 decode over histories whose row scales differ widely inside one attention split.

The reference quantiser (src/mla_compressed_q8_state.c:34-55) gives each row the scale
absmax/127. After RMSNorm a row's absmax ranges from its RMS (a flat row, all entries of one
magnitude) to sqrt(R) times its RMS (a one-hot-like row), and an all-zero latent (a zero hidden
state) is stored with scale 1 and zero codes. The GPU kernel quantises its softmax-weighted
mix against the largest scale of each split, so these rows stress its precision; the
reference accumulates in double and has no such dependence.

Histories of 8192 and 32768 rows mix Gaussian rows with one-hot-like rows every 61 rows, flat
rows every 97 rows, one all-zero row and one row 10x larger than the rest. The one-hot-like
rows sit at the latent column where the query's absorbed heads are largest ("favoured": their
logits are the largest of the history) or smallest ("suppressed"), with sharp attention (q_proj
std 0.16). Each decode is compared with the oracle (the reference's arithmetic) on identical
rows: max|got - ref| / max|ref| <= 2e-3.
"""
import ctypes as C

import numpy as np
import pytest

import pyoracle
from helpers import Api, f32, i8, rel_err, u16
from kvl_mla import abi, inputs, lib

pytestmark = pytest.mark.gpu

TOL = 2e-3
ORC = pyoracle.load_oracle()
O = Api(ORC, "orc_")
L = lib.load()
G = Api(L, "kvl_")


def pack_rows(lat, rope_raw, theta):
    """Reference quantiser + RoPE at the row position + BF16 (the oracle's restatement)."""
    n, R = lat.shape
    DR = rope_raw.shape[1]
    codes = np.zeros((n, R), np.int8)
    scl = np.zeros(n, np.float32)
    rb = np.zeros((n, DR), np.uint16)
    for i in range(n):
        ORC.orc_q8_pack_row(i8(codes[i]), f32(scl[i:i + 1]), u16(rb[i]), f32(lat[i]), f32(rope_raw[i]),
                            R, DR, i, np.float32(theta))
    return codes, scl, rb


def absorbed_query(cfg, layer, x):
    """q_lat[h] = W_UK[h]^T q_nope[h] in float64 (direction only: picks the one-hot column)."""
    NH, DN, DR, R = cfg.num_heads, cfg.qk_nope_dim, cfg.qk_rope_dim, cfg.kv_lora_rank
    f = lambda a: inputs.bf16_bits_to_f32(a).astype(np.float64)  # noqa: E731
    q = (f(layer.q_proj) @ x.astype(np.float64)).reshape(NH, DN + DR)
    wb = f(layer.kv_b_proj).reshape(NH, DN + cfg.v_head_dim, R)
    return np.stack([wb[h, :DN].T @ q[h, :DN] for h in range(NH)])  # [NH, R]


def history(n, R, DR, seed, col, sign):
    lat = inputs.normal_f32(seed, "lat", (n, R))
    rope = inputs.normal_f32(seed, "rope", (n, DR))
    for i in range(3, n, 61):                       # one-hot-like: absmax = sqrt(R) x RMS
        lat[i] = 0.0
        lat[i, col] = np.float32(sign * np.sqrt(R))
        lat[i, (col + 1 + i) % R] = np.float32(1e-3)  # not exactly one-hot
    for i in range(7, n, 97):                       # flat: absmax = RMS
        lat[i] = np.where(inputs.normal_f32(seed + i, "s", (R,)) >= 0, 1.0, -1.0).astype(np.float32)
    lat[n // 3] = 0.0                               # zero latent -> scale 1, zero codes
    lat[(2 * n) // 3] *= np.float32(10.0)           # one large row
    return np.ascontiguousarray(lat), np.ascontiguousarray(rope)


@pytest.mark.parametrize("n", [8192, 32768])
@pytest.mark.parametrize("mode", ["favoured", "suppressed"])
def test_q8_decode_heterogeneous_row_scales(n, mode):
    print(f"[q8-scales] rows {n} one-hot rows {mode}", flush=True)
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.make_layer(cfg, 0xE1, q_std=0.16)
    w = layer.struct()
    R, DR = cfg.kv_lora_rank, cfg.qk_rope_dim
    x = inputs.hidden(cfg, 0xE1, 1, tag="query")[0]
    qlat = absorbed_query(cfg, layer, x).sum(axis=0)
    col = int(np.argmax(np.abs(qlat)))
    sign = float(np.sign(qlat[col])) * (1.0 if mode == "favoured" else -1.0)
    lat, rope = history(n, R, DR, 0xE2 + n, col, sign)
    codes, scl, rb = pack_rows(lat, rope, cfg.rope_theta)
    assert scl[n // 3] == 1.0 and not codes[n // 3].any()
    print(f"[q8-scales]   scales: min {scl.min():.3e} max {scl.max():.3e} (one-hot {scl[3]:.3e})", flush=True)
    outs = []
    for api in (G, O):
        st = abi.KvlMlaCompressedQ8State()
        assert api.mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), n + 1) == 0
        np.ctypeslib.as_array(st.latent_q8, ((n + 1) * R,))[:n * R] = codes.ravel()
        np.ctypeslib.as_array(st.latent_scale, (n + 1,))[:n] = scl
        np.ctypeslib.as_array(st.rope_bf16, ((n + 1) * DR,))[:n * DR] = rb.ravel()
        st.len = n
        out = np.zeros(cfg.hidden_size, np.float32)
        assert api.mla_decode_compressed_q8_bf16(f32(out), f32(x), n, C.byref(cfg), C.byref(w), C.byref(st)) == 0
        outs.append(out)
        api.mla_compressed_q8_state_free(C.byref(st))
    e = rel_err(outs[0], outs[1])
    print(f"[q8-scales]   max|d|/max|ref| = {e:.3e}", flush=True)
    assert e <= TOL, e
