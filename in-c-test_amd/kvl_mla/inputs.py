"""Seeded synthetic inputs for the MLA path (weights, hidden states, latent histories).

SplitMix64 -> Box-Muller (float64) -> float32, optionally rounded to BF16 with
round-to-nearest-even. Every tensor is derived from (seed, tensor tag) so tests, the bench and
the CPU baseline see bit-identical inputs. Shapes follow the reference's KvlMlaConfig /
KvlMlaBF16 contract (include/kvl/ops.h:17-34): row-major [out, in] BF16 matrices.
"""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import abi

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

# Kimi-VL MLA shapes (hidden 2048, 16 heads, kv_lora_rank 512, nope 128, rope 64, v 128)
KIMI = dict(hidden_size=2048, num_heads=16, qk_nope_dim=128, qk_rope_dim=64, v_head_dim=128,
            kv_lora_rank=512, rms_eps=1e-5, rope_theta=50000.0)


def splitmix64(seed, n):
    """n consecutive SplitMix64 outputs of the stream starting at ``seed``."""
    with np.errstate(over="ignore"):
        k = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed) + k * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed, n, mean=0.0, std=1.0):
    """float64 N(mean, std^2) samples (Box-Muller on pairs of 53-bit uniforms)."""
    m = (n + 1) // 2
    r = splitmix64(seed, 2 * m)
    u1 = ((r[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) / 9007199254740992.0
    u2 = (r[1::2] >> np.uint64(11)).astype(np.float64) / 9007199254740992.0
    rad = np.sqrt(-2.0 * np.log(u1))
    ang = 2.0 * np.pi * u2
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = rad * np.cos(ang)
    z[1::2] = rad * np.sin(ang)
    return mean + std * z[:n]


def f32_to_bf16_bits(x):
    """float32 -> BF16 bits with the runtime's RNE rule (Inf/NaN truncated)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    finite = (u & np.uint32(0x7F800000)) != np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = np.where(finite, u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)), u)
    return (r >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def tag_seed(seed, tag):
    """Independent stream per (seed, tag)."""
    h = np.uint64(seed) ^ np.uint64(int.from_bytes(tag.encode()[:8].ljust(8, b"\0"), "little"))
    return int(splitmix64(int(h), 1)[0])


def normal_f32(seed, tag, shape, mean=0.0, std=1.0):
    n = int(np.prod(shape))
    return normal(tag_seed(seed, tag), n, mean, std).astype(np.float32).reshape(shape)


def normal_bf16(seed, tag, shape, mean=0.0, std=1.0):
    return f32_to_bf16_bits(normal_f32(seed, tag, shape, mean, std))


def config(**over):
    d = dict(KIMI)
    d.update(over)
    return abi.KvlMlaConfig(**d)


@dataclass
class Layer:
    """BF16 weights of one MLA layer plus the KvlMlaBF16 view the C API takes."""
    q_proj: np.ndarray
    kv_a_proj: np.ndarray
    kv_a_norm: np.ndarray
    kv_b_proj: np.ndarray
    o_proj: np.ndarray

    def struct(self):
        u16 = C.c_uint16
        return abi.KvlMlaBF16(abi.ptr(self.q_proj, u16), abi.ptr(self.kv_a_proj, u16),
                              abi.ptr(self.kv_a_norm, u16), abi.ptr(self.kv_b_proj, u16),
                              abi.ptr(self.o_proj, u16))


def make_layer(cfg, seed, std=0.02, q_std=None):
    """Random-init layer: matrices bf16(N(0, std)), kv_a_norm bf16(1 + N(0, std)). q_std (default
    std) scales q_proj alone: larger values give larger attention logits (sharper softmax)."""
    H, NH = cfg.hidden_size, cfg.num_heads
    DN, DR, DV, R = cfg.qk_nope_dim, cfg.qk_rope_dim, cfg.v_head_dim, cfg.kv_lora_rank
    return Layer(q_proj=normal_bf16(seed, "q_proj", (NH * (DN + DR), H), std=std if q_std is None else q_std),
                 kv_a_proj=normal_bf16(seed, "kv_a", (R + DR, H), std=std),
                 kv_a_norm=normal_bf16(seed, "kv_norm", (R,), mean=1.0, std=std),
                 kv_b_proj=normal_bf16(seed, "kv_b", (NH * (DN + DV), R), std=std),
                 o_proj=normal_bf16(seed, "o_proj", (H, NH * DV), std=std))


def fast_layer(cfg, seed):
    """Random-init layer drawn with numpy's PCG64 (fast enough for 27-layer stacks):
    bf16(N(0, 0.02)) matrices and bf16(1 + N(0, 0.02)) kv_a_norm, in a fixed draw order."""
    rng = np.random.default_rng(seed)
    H, NH = cfg.hidden_size, cfg.num_heads
    DN, DR, DV, R = cfg.qk_nope_dim, cfg.qk_rope_dim, cfg.v_head_dim, cfg.kv_lora_rank

    def mat(shape, mean=0.0):
        return f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)
                                + np.float32(mean))
    return Layer(q_proj=mat((NH * (DN + DR), H)), kv_a_proj=mat((R + DR, H)), kv_a_norm=mat((R,), 1.0),
                 kv_b_proj=mat((NH * (DN + DV), R)), o_proj=mat((H, NH * DV)))


def stack_seed(layer, seq):
    """Seed of the synthetic Q8 history of (layer, sequence) in the 27-layer stack workload."""
    return (0xC4 << 16) ^ (layer << 8) ^ seq


def hidden(cfg, seed, n, bf16_exact=False, tag="x"):
    """[n, hidden] float32 hidden states ~ N(0,1); optionally BF16-representable."""
    x = normal_f32(seed, tag, (n, cfg.hidden_size))
    return bf16_bits_to_f32(f32_to_bf16_bits(x)) if bf16_exact else x


def synth_normal(seed, idx):
    """Host mirror of the device history generator: approx. N(0,1) as the Irwin-Hall sum of
    four 24-bit uniforms (SplitMix64 outputs 4*idx+1 .. 4*idx+4), centred, times sqrt(3).
    Only exactly rounded float32 operations, so it matches the device bit for bit."""
    idx = np.asarray(idx, dtype=np.uint64)
    k = idx[..., None] * np.uint64(4) + np.arange(1, 5, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + k * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    u = (z >> np.uint64(40)).astype(np.float32) * np.float32(5.9604644775390625e-8)
    s = (u[..., 0] + u[..., 1]) + (u[..., 2] + u[..., 3])
    return ((s - np.float32(2.0)) * np.float32(1.7320508)).astype(np.float32)


def synth_rows(seed, rows, R, DR):
    """Raw synthetic history rows (float32 latent [n, R] and RoPE key [n, DR]) of the given
    global row indices, as the device generator draws them."""
    rows = np.asarray(rows, dtype=np.uint64)
    base = rows[:, None] * np.uint64(R + DR)
    lat = synth_normal(seed, base + np.arange(R, dtype=np.uint64))
    rope = synth_normal(seed, base + np.uint64(R) + np.arange(DR, dtype=np.uint64))
    return lat, rope
