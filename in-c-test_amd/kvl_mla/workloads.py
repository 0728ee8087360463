"""Workload drivers for profiling the library's launches in isolation (rocprofv3 kernel traces
and counters): each runs one workload a given number of times on synthetic, seeded data.

    python3 in-c-test_amd/kvl_mla/workloads.py block  [--kind q8|bf16] [--ctx 32768] [--tokens 8] [--reps 10]
    python3 in-c-test_amd/kvl_mla/workloads.py single [--kind q8|bf16] [--ctx 32768] [--reps 10]
    python3 in-c-test_amd/kvl_mla/workloads.py ragged [--kind bf16|f32] [--reps 20]

block:  a block decode of `tokens` draft tokens over one sequence's history (host API), the
        state truncated back after each call (src/mla_compressed_state.c:163-184);
single: one single-token decode over the same history (host API);
ragged: one decode token for each of 64 sequences with histories of 512..32768 rows (seeded),
        batched device API with KVL_MLA_NO_ADVANCE.
Each prints one line with the median host time per call.
"""
import argparse
import ctypes as C
import os
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import numpy as np  # noqa: E402

from kvl_mla import abi, inputs, lib  # noqa: E402

STATES = {
    "q8": (abi.KvlMlaCompressedQ8State, "compressed_q8_state", "mla_decode_compressed_q8_bf16",
           "mla_decode_compressed_q8_block_bf16", None),
    "bf16": (abi.KvlMlaCompressedBF16State, "compressed_bf16_state", "mla_decode_compressed_bf16_bf16",
             "mla_decode_compressed_bf16_block_bf16", "mla_decode_compressed_bf16_batch_device"),
    "f32": (abi.KvlMlaCompressedState, "compressed_state", "mla_decode_compressed_bf16",
            "mla_decode_compressed_block_bf16", "mla_decode_compressed_batch_device"),
}


def f32p(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def median_ms(fn, reps):
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2] * 1e3


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("workload", choices=["block", "single", "ragged"])
    ap.add_argument("--kind", default=None)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--tokens", type=int, default=8)
    ap.add_argument("--reps", type=int, default=10)
    args = ap.parse_args()
    kind = args.kind or ("bf16" if args.workload == "ragged" else "q8")
    L = lib.load()
    cfg = inputs.config(**inputs.KIMI)
    layer = inputs.fast_layer(cfg, 0xB5)
    w = layer.struct()
    lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(w)), "bind")
    T, name, single, block, batch = STATES[kind]
    init = getattr(L, f"kvl_mla_{name}_init")
    fill = getattr(L, f"kvl_mla_{name}_fill_synthetic")
    free = getattr(L, f"kvl_mla_{name}_free")
    if args.workload in ("block", "single"):
        st = T()
        lib.check(init(C.byref(st), C.byref(cfg), args.ctx + args.tokens + 1), "init")
        lib.check(fill(C.byref(st), 0, args.ctx, 0xB5), "fill")
        x = np.ascontiguousarray(inputs.hidden(cfg, 0xB5, args.tokens, tag="block_x"))
        out = np.zeros_like(x)
        trunc = getattr(L, f"kvl_mla_{name}_truncate")
        if args.workload == "block":
            def call():
                lib.check(getattr(L, "kvl_" + block)(f32p(out), f32p(x), args.tokens, args.ctx, C.byref(cfg),
                                                     C.byref(w), C.byref(st)), "block")
                lib.check(trunc(C.byref(st), args.ctx), "truncate")
        else:
            def call():
                lib.check(getattr(L, "kvl_" + single)(f32p(out[0]), f32p(x[0]), args.ctx, C.byref(cfg), C.byref(w),
                                                      C.byref(st)), "single")
                lib.check(trunc(C.byref(st), args.ctx), "truncate")
        call()
        ms = median_ms(call, args.reps)
        print(f"{args.workload} {kind} ctx={args.ctx} tokens={args.tokens if args.workload == 'block' else 1}: "
              f"median {ms:.4f} ms per call", flush=True)
        free(C.byref(st))
        return
    if batch is None:
        raise SystemExit("ragged: kind bf16 or f32")
    lens = np.random.default_rng(0xC8).integers(512, 32769, size=64)
    sts = []
    for i, n in enumerate(lens):
        st = T()
        lib.check(init(C.byref(st), C.byref(cfg), int(n) + 1), "init")
        lib.check(fill(C.byref(st), 0, int(n), 0xC80 + i), "fill")
        sts.append(st)
    arr = (C.POINTER(T) * len(sts))(*[C.pointer(s) for s in sts])
    x = np.ascontiguousarray(inputs.hidden(cfg, 0xC8, len(sts), tag="query"))
    dx, do = L.kvl_mla_device_alloc(x.nbytes), L.kvl_mla_device_alloc(x.nbytes)
    lib.check(L.kvl_mla_copy_to_device(dx, x.ctypes.data, x.nbytes), "h2d")
    dec = getattr(L, "kvl_" + batch)

    def call():
        lib.check(dec(do, dx, len(sts), C.byref(cfg), C.byref(w), arr, lib.NO_ADVANCE), "ragged")
        lib.check(L.kvl_mla_synchronize(), "sync")
    call()
    ms = median_ms(call, args.reps)
    print(f"ragged {kind} 64 sequences ({int(lens.sum())} rows): median {ms:.4f} ms per call", flush=True)
    L.kvl_mla_device_free(dx)
    L.kvl_mla_device_free(do)
    for st in sts:
        free(C.byref(st))


if __name__ == "__main__":
    main()
