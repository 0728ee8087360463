"""CPU checks of the drop-in boundary: libkvl_mla loads, exports every function that
include/kvl/*.h declares, and its structs have the reference's byte layout. No GPU call."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from kvl_mla import abi, inputs, lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include", "kvl")
REF_INCLUDE = "/root/reference/include"


def declared_functions():
    names = set()
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z][\w \*]*?\b(kvl_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_function():
    L = lib.load()  # dlopen only: no HIP call is made
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing


def test_reference_api_symbols_declared():
    # every symbol of the reference MLA API (include/kvl/ops.h:43-64, mla_state.h:24-37,
    # mla_compressed_state.h:16-44, mla_compressed_q8_state.h:18-38) is part of the boundary
    names = declared_functions()
    for n in list(abi.REFERENCE_API) + list(abi.PREFILL_API):
        assert "kvl_" + n in names, n


def test_struct_sizes_ctypes():
    assert C.sizeof(abi.KvlMlaConfig) == 32
    assert C.sizeof(abi.KvlMlaBF16) == 40
    assert C.sizeof(abi.KvlMlaState) == 40
    assert C.sizeof(abi.KvlMlaCompressedState) == 32
    assert C.sizeof(abi.KvlMlaCompressedQ8State) == 40
    # the BF16-latent extension state: the FP32 state's layout with bf16 arrays
    assert C.sizeof(abi.KvlMlaCompressedBF16State) == 32
    assert abi.KvlMlaCompressedBF16State.rope.offset == abi.KvlMlaCompressedState.rope.offset == 24


LAYOUT_C = r"""
#include <stdio.h>
#include <stddef.h>
#include "kvl/ops.h"
#include "kvl/mla_state.h"
#include "kvl/mla_compressed_state.h"
#include "kvl/mla_compressed_q8_state.h"
#define P(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  printf("cfg %zu bf16 %zu st %zu cs %zu q8 %zu\n", sizeof(KvlMlaConfig), sizeof(KvlMlaBF16),
         sizeof(KvlMlaState), sizeof(KvlMlaCompressedState), sizeof(KvlMlaCompressedQ8State));
  P(KvlMlaConfig, rope_theta) P(KvlMlaBF16, o_proj) P(KvlMlaState, values)
  P(KvlMlaCompressedState, rope) P(KvlMlaCompressedQ8State, rope_bf16)
  P(KvlMlaCompressedQ8State, latent_scale) P(KvlMlaState, v_head_dim)
  return 0;
}
"""


def _layout(include_dir, tmp_path, tag):
    src = tmp_path / f"layout_{tag}.c"
    exe = tmp_path / f"layout_{tag}"
    src.write_text(LAYOUT_C)
    subprocess.run(["gcc", "-std=c11", "-I", include_dir, str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout


def test_struct_layout_matches_reference_headers(tmp_path):
    if not os.path.isdir(REF_INCLUDE):
        pytest.skip("reference headers not present")
    ours = _layout(os.path.join(ROOT, "include"), tmp_path, "ours")
    ref = _layout(REF_INCLUDE, tmp_path, "ref")
    assert ours == ref


def test_synth_normal_moments_and_determinism():
    v = inputs.synth_normal(0xC4, np.arange(400000))
    assert abs(float(v.mean())) < 0.01 and abs(float(v.std()) - 1.0) < 0.01
    assert np.max(np.abs(v)) <= 2.0 * np.sqrt(3.0)
    np.testing.assert_array_equal(v[1000:1010], inputs.synth_normal(0xC4, np.arange(1000, 1010)))


def test_host_helpers_match_reference_formulas():
    """The library's host-only exports, called through the C ABI (no HIP call is made):
    kvl_bf16_to_f32 over every BF16 word is the word shifted into the high half
    (src/ops.c:12-17); the *_state_bytes of the three state kinds are sizeof(struct) plus
    capacity x the per-row bytes of the reference layouts (src/mla_state.c:57-64,
    src/mla_compressed_state.c:47-50, src/mla_compressed_q8_state.c:104-109; the BF16-latent
    extension state: 2 bytes per element, 1152 B per row at the Kimi dims), and 0 for a freed
    state."""
    L = lib.load()
    words = np.arange(65536, dtype=np.uint32)
    got = np.array([L.kvl_bf16_to_f32(int(u)) for u in words], dtype=np.float32)
    want = words << np.uint32(16)
    # ctypes returns the float as a Python float (a double): signalling NaNs come back quieted,
    # so NaN words are checked as NaN with the same sign, every other word bit for bit
    nan = np.isnan(want.view(np.float32))
    np.testing.assert_array_equal(got.view(np.uint32)[~nan], want[~nan])
    assert np.isnan(got[nan]).all()
    np.testing.assert_array_equal(np.signbit(got[nan]), np.signbit(want.view(np.float32)[nan]))
    for d, cap in ((dict(inputs.KIMI), 33), (dict(inputs.KIMI, num_heads=4, kv_lora_rank=96, qk_rope_dim=16), 7)):
        cfg = inputs.config(**d)
        R, DR, NH = cfg.kv_lora_rank, cfg.qk_rope_dim, cfg.num_heads
        QD, DV = cfg.qk_nope_dim + cfg.qk_rope_dim, cfg.v_head_dim
        cases = ((abi.KvlMlaCompressedQ8State, "compressed_q8_state", R + 4 + 2 * DR),
                 (abi.KvlMlaCompressedState, "compressed_state", 4 * (R + DR)),
                 (abi.KvlMlaState, "state", 4 * NH * (QD + DV)),
                 (abi.KvlMlaCompressedBF16State, "compressed_bf16_state", 2 * (R + DR)))
        for T, name, per_row in cases:
            st = T()
            assert getattr(L, f"kvl_mla_{name}_init")(C.byref(st), C.byref(cfg), cap) == 0
            assert getattr(L, f"kvl_mla_{name}_bytes")(C.byref(st)) == C.sizeof(T) + cap * per_row, name
            getattr(L, f"kvl_mla_{name}_free")(C.byref(st))
            assert getattr(L, f"kvl_mla_{name}_bytes")(C.byref(st)) == 0, name


def test_bf16_state_life_cycle_checks():
    """The BF16-latent state keeps the FP32 state's argument rules (src/mla_compressed_state.c:
    24-50): init rejects an odd qk_rope_dim or capacity <= 0, truncate only shortens, reset empties.
    Host-only calls (no HIP call is made)."""
    L = lib.load()
    cfg = inputs.config(**inputs.KIMI)
    st = abi.KvlMlaCompressedBF16State()
    assert L.kvl_mla_compressed_bf16_state_init(C.byref(st), C.byref(cfg), 0) == -1
    odd = inputs.config(**dict(inputs.KIMI, qk_rope_dim=63))
    assert L.kvl_mla_compressed_bf16_state_init(C.byref(st), C.byref(odd), 8) == -1
    assert L.kvl_mla_compressed_bf16_state_init(C.byref(st), C.byref(cfg), 8) == 0
    assert (st.capacity, st.len, st.kv_lora_rank, st.qk_rope_dim) == (8, 0, 512, 64)
    assert L.kvl_mla_compressed_bf16_state_truncate(C.byref(st), 1) == -1
    st.len = 5
    assert L.kvl_mla_compressed_bf16_state_truncate(C.byref(st), 3) == 0 and st.len == 3
    assert L.kvl_mla_compressed_bf16_state_truncate(C.byref(st), -1) == -1
    L.kvl_mla_compressed_bf16_state_reset(C.byref(st))
    assert st.len == 0
    L.kvl_mla_compressed_bf16_state_free(C.byref(st))
    assert st.capacity == 0 and not st.latent and not st.rope
