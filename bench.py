#!/usr/bin/env python3
"""Benchmark of the MI355X MLA library on its headline workload.

Workload (one "step"): one decode token through a 27-layer MLA attention stack (q_proj,
kv_a_proj + RMSNorm, absorbed kv_b_proj, o_proj, residual; no MoE) for a batch of 8
sequences, each holding a 32768-token row-wise Q8 latent history per layer (512 int8 + fp32
scale + 64 bf16 RoPE key = 644 B/token). Weights are random-init bf16 N(0, 0.02), histories
are generated on the device (synthetic), all resident in HBM before timing. Every step
appends at position 32768 without advancing, so steps are identical.

value = algorithmic bytes of a step (weights once per layer + every history row read once)
        / wall-clock time per step, in GB/s.
Also reported: the attention kernel's roofline (HIP events on the library stream, recorded
inside a replay of the step graph; eager-launch events beside them), the stage breakdown, causal prefill TFLOP/s at 4096 tokens, and a CPU baseline (the reference
C path compiled from its sources when available, else the oracle) on a bounded sample,
whose outputs double as a parity check of the benchmark workload.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "in-c-test_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

from kvl_mla import abi, inputs, lib  # noqa: E402

METRIC = "MLA decode HBM GB/s (% peak) @32K ctx Q8 cache; prefill TFLOP/s @4K"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
Q8_ROW = 512 + 4 + 2 * 64


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(cfg):
    H, NH = cfg.hidden_size, cfg.num_heads
    DN, DR, DV, R = cfg.qk_nope_dim, cfg.qk_rope_dim, cfg.v_head_dim, cfg.kv_lora_rank
    return 2 * (NH * (DN + DR) * H + (R + DR) * H + R + NH * (DN + DV) * R + H * NH * DV)


def prefill_flops(S, cfg):
    """Algorithmic flops of the reference's non-absorbed causal prefill
    (src/mla_prefill_streaming.c:78-206): kv_a, q, kv_b expansion, QK^T and PV over the
    S(S+1)/2 causal pairs, o_proj. Softmax, RMSNorm and RoPE excluded."""
    H, NH = cfg.hidden_size, cfg.num_heads
    DN, DR, DV, R = cfg.qk_nope_dim, cfg.qk_rope_dim, cfg.v_head_dim, cfg.kv_lora_rank
    pairs = S * (S + 1) // 2
    return (2 * S * H * (R + DR) + 2 * S * H * NH * (DN + DR) + 2 * S * R * NH * (DN + DV)
            + 2 * NH * pairs * (DN + DR) + 2 * NH * pairs * DV + 2 * S * NH * DV * H)


def omp_threads():
    try:
        return int(C.CDLL("libgomp.so.1").omp_get_max_threads())
    except OSError:
        return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def traffic_bytes(batch, context):
    """HBM bytes per attention launch measured by rocprofv3 (FETCH_SIZE and WRITE_SIZE passes,
    scaled by a copy kernel of known size) for this workload, from the committed profile;
    None for other workloads."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "k_attn_q8_mfma_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("workload") != {"batch": batch, "context": context}:
        return None
    return t.get("hbm_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=27)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--prefill-tokens", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-block", action="store_true", help="skip the block-verify leg")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run a plain copy kernel of MIB MiB (memory-counter calibration)")
    ap.add_argument("--no-ragged", action="store_true", help="skip the 64-sequence ragged decode leg")
    ap.add_argument("--no-peak", action="store_true", help="skip the measured copy-bandwidth leg")
    ap.add_argument("--no-batch1", action="store_true", help="skip the batch-1 decode legs (config 0 and 1)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the MLA path here runs on a single GPU "
              "(multi-GPU sharding is a design note, not part of this build); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    L = lib.load()
    lib.check(L.kvl_mla_init(), "init")
    cfg = inputs.config(**inputs.KIMI)
    NL, B, CTX = args.layers, args.batch, args.context
    H = cfg.hidden_size

    t_setup = time.time()
    layers, wstructs = [], []
    for li in range(NL):
        lw = inputs.fast_layer(cfg, 0xC4 + li)
        layers.append(lw)
        ws = lw.struct()
        wstructs.append(ws)
        lib.check(L.kvl_mla_bind_weights(C.byref(cfg), C.byref(ws)), "bind weights")
    log(f"[bench] weights bound ({NL} layers) in {time.time() - t_setup:.1f}s")
    Q8P = C.POINTER(abi.KvlMlaCompressedQ8State)
    states, arrays = [], []
    for li in range(NL):
        row = []
        for b in range(B):
            st = abi.KvlMlaCompressedQ8State()
            if L.kvl_mla_compressed_q8_state_init(C.byref(st), C.byref(cfg), CTX + 1) != 0:
                raise RuntimeError("state init failed")
            lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, CTX, inputs.stack_seed(li, b)),
                      "fill")
            row.append(st)
        states.append(row)
        arrays.append((Q8P * B)(*[C.pointer(s) for s in row]))
    log(f"[bench] {NL * B} Q8 histories of {CTX} tokens generated in {time.time() - t_setup:.1f}s")

    x0 = np.ascontiguousarray(inputs.hidden(cfg, 0xC4, B, tag="stack_x"))
    nbytes = x0.nbytes
    d_x0 = L.kvl_mla_device_alloc(nbytes)
    d_h = L.kvl_mla_device_alloc(nbytes)
    d_l0 = L.kvl_mla_device_alloc(nbytes)
    if not (d_x0 and d_h and d_l0):
        raise RuntimeError("device alloc failed: " + lib.last_error())
    lib.check(L.kvl_mla_copy_to_device(d_x0, x0.ctypes.data, nbytes), "h2d")
    flags = lib.RESIDUAL | lib.NO_ADVANCE

    def step():
        lib.check(L.kvl_mla_copy_kernel(d_h, d_x0, nbytes), "reset hidden")
        for li in range(NL):
            rc = L.kvl_mla_decode_compressed_q8_batch_device(d_h, d_h, B, C.byref(cfg), C.byref(wstructs[li]),
                                                              arrays[li], flags)
            if rc != 0:
                raise RuntimeError("decode: " + lib.last_error())

    for _ in range(max(1, args.warmup)):
        step()
    lib.check(L.kvl_mla_synchronize(), "sync")

    # stage breakdown from events around each launch of eager steps (the graph-mode breakdown,
    # which the roofline uses, is taken after the timed region)
    lib.check(L.kvl_mla_timing_enable(1), "timing on")
    n_prof = 3
    for _ in range(n_prof):
        step()
    lib.check(L.kvl_mla_synchronize(), "sync")
    ms = (C.c_double * 6)()
    cnt = (C.c_int * 6)()
    lib.check(L.kvl_mla_timing_read(ms, cnt), "timing read")
    lib.check(L.kvl_mla_timing_enable(0), "timing off")
    stages = {name: {"ms_per_launch": ms[i] / max(cnt[i], 1), "launches": cnt[i]}
              for i, name in enumerate(lib.STAGES)}

    graph = None
    if not args.eager:
        lib.check(L.kvl_mla_capture_begin(), "capture begin")
        try:
            step()
        finally:
            ge = C.c_void_p()
            rc = L.kvl_mla_capture_end(C.byref(ge))
        lib.check(rc, "capture end")
        graph = ge
        for _ in range(max(1, args.warmup)):
            lib.check(L.kvl_mla_graph_launch(graph), "graph launch")
        lib.check(L.kvl_mla_synchronize(), "sync")

    K = args.steps
    lib.check(L.kvl_mla_synchronize(), "sync")
    t0 = time.perf_counter()
    e0 = L.kvl_mla_event_record()
    for _ in range(K):
        if graph is not None:
            lib.check(L.kvl_mla_graph_launch(graph), "graph launch")
        else:
            step()
    e1 = L.kvl_mla_event_record()
    lib.check(L.kvl_mla_synchronize(), "sync")
    t1 = time.perf_counter()
    ev_ms = L.kvl_mla_event_elapsed_ms(e0, e1) / K
    L.kvl_mla_event_destroy(e0)
    L.kvl_mla_event_destroy(e1)
    ms_step = (t1 - t0) * 1e3 / K
    # the per-step distribution: K more steps with an event recorded between consecutive steps
    evs = [L.kvl_mla_event_record()]
    for _ in range(K):
        if graph is not None:
            lib.check(L.kvl_mla_graph_launch(graph), "graph launch")
        else:
            step()
        evs.append(L.kvl_mla_event_record())
    lib.check(L.kvl_mla_synchronize(), "sync")
    per_step = np.array([L.kvl_mla_event_elapsed_ms(evs[i], evs[i + 1]) for i in range(K)])
    for e in evs:
        L.kvl_mla_event_destroy(e)
    step_stats = {"mean": round(float(per_step.mean()), 4), "median": round(float(np.median(per_step)), 4),
                  "p10": round(float(np.percentile(per_step, 10)), 4),
                  "p90": round(float(np.percentile(per_step, 90)), 4), "steps": K,
                  "timing": "HIP events between consecutive steps (a second run of K steps)"}
    wb = weight_bytes(cfg)
    hist_bytes = B * (CTX + 1) * Q8_ROW
    step_bytes = NL * (wb + hist_bytes)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"[bench] step {ms_step:.3f} ms wall ({ev_ms:.3f} ms events), {value:.1f} GB/s; per step median "
        f"{step_stats['median']:.4f} ms, p10 {step_stats['p10']:.4f}, p90 {step_stats['p90']:.4f}")

    # the same step captured again with the stage events inside the graph (event-record
    # nodes): after a few replays, each layer's stage durations as the graph runs them
    eager_stages = stages
    timing_source = "events around eager launches"
    if graph is not None:
        lib.check(L.kvl_mla_timing_enable(2), "timing on (graph)")
        lib.check(L.kvl_mla_capture_begin(), "capture begin")
        try:
            step()
        finally:
            tg = C.c_void_p()
            rc = L.kvl_mla_capture_end(C.byref(tg))
        lib.check(L.kvl_mla_timing_enable(0), "timing off")
        if rc == 0:
            for _ in range(3):
                lib.check(L.kvl_mla_graph_launch(tg), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            rc = L.kvl_mla_timing_read(ms, cnt)
            L.kvl_mla_graph_destroy(tg)
        else:
            L.kvl_mla_timing_read(ms, cnt)  # drop the records of the failed capture
        if rc == 0:
            stages = {name: {"ms_per_launch": ms[i] / max(cnt[i], 1), "launches": cnt[i]}
                      for i, name in enumerate(lib.STAGES)}
            timing_source = "events recorded inside the step graph (last of 3 replays)"
        else:
            log(f"[bench] graph-mode stage timing unavailable ({lib.last_error()}); eager events used")

    # the roofline's launch time: the attention stage of the step graph carrying every stage's
    # event records (closest to the kernel trace: the records add their gaps). Also measured:
    # the attention launches alone bracketed (the other stages without records), which adds more
    # to the launch (its opening record waits on the previous kernel's end), reported beside it.
    attn_ms, attn_src = stages["attention"]["ms_per_launch"], timing_source
    attn_only_ms = None
    if graph is not None:
        lib.check(L.kvl_mla_timing_stages(1 << lib.STAGES.index("attention")), "timing mask")
        lib.check(L.kvl_mla_timing_enable(2), "timing on (graph)")
        lib.check(L.kvl_mla_capture_begin(), "capture begin")
        try:
            step()
        finally:
            tg = C.c_void_p()
            rc = L.kvl_mla_capture_end(C.byref(tg))
        lib.check(L.kvl_mla_timing_enable(0), "timing off")
        lib.check(L.kvl_mla_timing_stages(0x3F), "timing mask")
        if rc == 0:
            for _ in range(3):
                lib.check(L.kvl_mla_graph_launch(tg), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            if L.kvl_mla_timing_read(ms, cnt) == 0 and cnt[3]:
                attn_only_ms = ms[3] / cnt[3]
            L.kvl_mla_graph_destroy(tg)
        else:
            L.kvl_mla_timing_read(ms, cnt)
    # The attention launch of this workload also computes the q_proj | kv_a projection
    # (kvl_mla_set_fused_projection), prepares the queries and appends the rows
    # (kvl_mla_set_fused_qprep) and combines the split partials (kvl_mla_set_fused_combine): its
    # algorithmic bytes are the history rows plus the projection weights, W_UK^T and W_UV, the
    # layer input x, the q_proj | kv_a partials it writes and reads back, the query operands and
    # rows it writes and the head outputs (fp32 and bf16 hi | lo). The split partials stay in the
    # L2 of the XCD that combines them and are not counted.
    H_, NH_, R_, DN_, DR_ = cfg.hidden_size, cfg.num_heads, cfg.kv_lora_rank, cfg.qk_nope_dim, cfg.qk_rope_dim
    QO_, KVO_, DV_ = NH_ * (DN_ + DR_), R_ + DR_, cfg.v_head_dim
    fused_extra = (2 * (QO_ + KVO_) * H_ + 4 * B * H_ + 2 * NH_ * R_ * DN_ + 2 * NH_ * R_ * DV_
                   + 2 * 4 * 4 * B * (QO_ + KVO_) + B * NH_ * (2 * R_ + 4 + 4 * DR_) + B * Q8_ROW
                   + B * NH_ * DV_ * (4 + 2 + 2))
    attn_bytes = hist_bytes + fused_extra
    attn_gbs = attn_bytes / (attn_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(attn_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_bytes(B, CTX),
                "kernel": "k_attn_q8_mfma<true, true, kCombXcd> (the q_proj | kv_a projection, the query "
                          "preparation, the row append, the attention and the combine of its sequences)",
                "algorithmic_bytes_per_launch": attn_bytes, "history_bytes_per_launch": hist_bytes,
                "avg_launch_ms": round(attn_ms, 5), "timing": attn_src}
    if attn_only_ms is not None:
        roofline["avg_launch_ms_attention_events_only"] = round(attn_only_ms, 5)

    # The step with the combine in a launch of its own (the query preparation still inside the
    # attention launch): its step time.
    sep_comb = None
    if graph is not None:
        prev_comb = L.kvl_mla_set_fused_combine(0)
        try:
            lib.check(L.kvl_mla_capture_begin(), "capture begin")
            try:
                step()
            finally:
                g4 = C.c_void_p()
                rc = L.kvl_mla_capture_end(C.byref(g4))
            lib.check(rc, "capture end (separate combine)")
            for _ in range(max(1, args.warmup)):
                lib.check(L.kvl_mla_graph_launch(g4), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            t0 = time.perf_counter()
            for _ in range(K):
                lib.check(L.kvl_mla_graph_launch(g4), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            sep_ms = (time.perf_counter() - t0) * 1e3 / K
            L.kvl_mla_graph_destroy(g4)
            sep_comb = {"ms_per_step": round(sep_ms, 4),
                        "kernels": "k_attn_q8_mfma<true, true> then k_combine_r512"}
            log(f"[bench] combine in its own launch: step {sep_ms:.3f} ms")
        finally:
            L.kvl_mla_set_fused_combine(prev_comb)
    if sep_comb is not None:
        roofline["separate_combine_form"] = sep_comb

    # The same step in the two-launch form (append + query preparation in a launch of their own,
    # then the attention alone, then the combine): its step time, and the attention kernel's rate
    # over the history bytes, from the stage events inside the step graph as above.
    two = None
    if graph is not None:
        prev_form = L.kvl_mla_set_fused_qprep(0)
        try:
            lib.check(L.kvl_mla_capture_begin(), "capture begin")
            try:
                step()
            finally:
                g2 = C.c_void_p()
                rc = L.kvl_mla_capture_end(C.byref(g2))
            lib.check(rc, "capture end (two-launch form)")
            for _ in range(max(1, args.warmup)):
                lib.check(L.kvl_mla_graph_launch(g2), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            t0 = time.perf_counter()
            for _ in range(K):
                lib.check(L.kvl_mla_graph_launch(g2), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            two_ms = (time.perf_counter() - t0) * 1e3 / K
            L.kvl_mla_graph_destroy(g2)
            lib.check(L.kvl_mla_timing_enable(2), "timing on (graph)")
            lib.check(L.kvl_mla_capture_begin(), "capture begin")
            try:
                step()
            finally:
                g3 = C.c_void_p()
                rc = L.kvl_mla_capture_end(C.byref(g3))
            lib.check(L.kvl_mla_timing_enable(0), "timing off")
            lib.check(rc, "capture end (two-launch form, stage events)")
            for _ in range(3):
                lib.check(L.kvl_mla_graph_launch(g3), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            lib.check(L.kvl_mla_timing_read(ms, cnt), "timing read")
            L.kvl_mla_graph_destroy(g3)
            st2 = {name: ms[i] / cnt[i] for i, name in enumerate(lib.STAGES) if cnt[i]}
            a2 = st2["attention"]
            two = {"ms_per_step": round(two_ms, 4), "attention_ms": round(a2, 5),
                   "append_qprep_ms": round(st2.get("append_qprep", 0.0), 5),
                   "attention_achieved": round(hist_bytes / (a2 * 1e-3) / 1e9, 1),
                   "attention_frac": round(hist_bytes / (a2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "kernel": "k_attn_q8_mfma<true, false>", "timing": "events recorded inside the step graph"}
            log(f"[bench] two-launch form: step {two_ms:.3f} ms; attention {a2 * 1e3:.2f} us "
                f"({two['attention_achieved']:.1f} GB/s), append + query prep {two['append_qprep_ms'] * 1e3:.2f} us")
        finally:
            L.kvl_mla_set_fused_qprep(prev_form)
    if two is not None:
        roofline["two_launch_form"] = two

    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"{NL}-layer MLA attention stack decode, batch {B}, {CTX}-token row-wise Q8 "
                               f"latent history per layer and sequence", "layers": NL, "batch": B,
                   "context": CTX, "hidden": H, "heads": cfg.num_heads, "kv_lora_rank": cfg.kv_lora_rank,
                   "qk_rope_dim": cfg.qk_rope_dim, "history_row_bytes": Q8_ROW,
                   "bytes_per_step": step_bytes, "mode": "eager" if graph is None else "hip-graph"},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "step_ms": step_stats,
        "roofline": roofline,
        "stages_ms_per_launch": {k: round(v["ms_per_launch"], 5) for k, v in stages.items() if v["launches"]},
        "stages_eager_ms_per_launch": {k: round(v["ms_per_launch"], 5) for k, v in eager_stages.items()
                                       if v["launches"]},
        "stages_note": "each stage launch bracketed by its own pair of event records, whose gaps the "
                       "durations include (they sum to more than the step); the kernel trace in profiles/ "
                       "gives the launches alone",
    }

    # ---- parity spot check + CPU baseline on layer 0 -------------------------------------
    lib.check(L.kvl_mla_decode_compressed_q8_batch_device(d_l0, d_x0, B, C.byref(cfg), C.byref(wstructs[0]),
                                                          arrays[0], lib.NO_ADVANCE), "layer-0 decode")
    gpu_l0 = np.zeros_like(x0)
    lib.check(L.kvl_mla_copy_to_host(gpu_l0.ctypes.data, d_l0, nbytes), "d2h")
    if not args.no_cpu:
        import pyoracle
        from helpers import rel_err
        ref = pyoracle.load_reference("avx2")
        kind = "reference" if ref is not None else "port"
        cpu = ref if ref is not None else pyoracle.load_oracle()
        fn = cpu.kvl_mla_decode_compressed_q8_bf16 if ref is not None else cpu.orc_mla_decode_compressed_q8_bf16
        errs, t_cpu, n_done = [], 0.0, 0
        for b in range(B):
            st = states[0][b]
            lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, CTX), "pull")
            out = np.zeros(H, np.float32)
            ts = time.perf_counter()
            rc = fn(out.ctypes.data_as(abi.f32p), x0[b].ctypes.data_as(abi.f32p), CTX, C.byref(cfg),
                    C.byref(wstructs[0]), C.byref(st))
            t_cpu += time.perf_counter() - ts
            st.len = CTX  # the CPU call appended at position CTX; restore
            if rc != 0:
                raise RuntimeError("CPU baseline call failed")
            errs.append(rel_err(gpu_l0[b], out))
            n_done += 1
            if t_cpu > 25.0:
                break
        sample_bytes = wb + n_done * (CTX + 1) * Q8_ROW
        result["cpu_baseline"] = {
            "value": round(sample_bytes / t_cpu / 1e9, 3), "unit": "GB/s", "cores": omp_threads(), "kind": kind,
            "sample": f"layer 0 of the stack, {n_done} of {B} sequences at {CTX} tokens, one decode token each "
                      f"({t_cpu:.2f} s; the reference loops its single-sequence API; attention loops are "
                      f"single-threaded there, GEMVs use OpenMP)"}
        result["parity"] = {"layer0_max_rel_err_vs_cpu": float(max(errs)), "tolerance": 2e-3,
                            "sequences": n_done}
        log(f"[bench] cpu baseline {result['cpu_baseline']['value']} GB/s ({kind}), parity {max(errs):.2e}")

    # ---- block verify: 8 draft tokens of one sequence over the 32K Q8 history of layer 0 ----
    # (host API both ways: one block call against 8 single-token decodes; equal bit for bit)
    if not args.no_block:
        T = 8
        bst = abi.KvlMlaCompressedQ8State()
        lib.check(L.kvl_mla_compressed_q8_state_init(C.byref(bst), C.byref(cfg), CTX + T), "block state init")
        lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(bst), 0, CTX, 0xB5), "block state fill")
        xb = np.ascontiguousarray(inputs.hidden(cfg, 0xB5, T, tag="block_x"))
        o_blk, o_ser = np.zeros_like(xb), np.zeros_like(xb)
        fp = lambda a: a.ctypes.data_as(abi.f32p)  # noqa: E731

        def serial():
            for t in range(T):
                lib.check(L.kvl_mla_decode_compressed_q8_bf16(fp(o_ser[t]), fp(xb[t]), CTX + t, C.byref(cfg),
                                                              C.byref(wstructs[0]), C.byref(bst)), "serial decode")
            lib.check(L.kvl_mla_compressed_q8_state_truncate(C.byref(bst), CTX), "truncate")

        def block():
            lib.check(L.kvl_mla_decode_compressed_q8_block_bf16(fp(o_blk), fp(xb), T, CTX, C.byref(cfg),
                                                                C.byref(wstructs[0]), C.byref(bst)), "block decode")
            lib.check(L.kvl_mla_compressed_q8_state_truncate(C.byref(bst), CTX), "truncate")

        def single():
            lib.check(L.kvl_mla_decode_compressed_q8_bf16(fp(o_ser[0]), fp(xb[0]), CTX, C.byref(cfg),
                                                          C.byref(wstructs[0]), C.byref(bst)), "single decode")
            lib.check(L.kvl_mla_compressed_q8_state_truncate(C.byref(bst), CTX), "truncate")

        times = {}
        for name, fn in (("single", single), ("serial", serial), ("block", block)):
            fn()
            reps = 10
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            times[name] = sorted(ts)[reps // 2] * 1e3  # median
        same = bool(np.array_equal(o_blk, o_ser))
        result["block_verify"] = {"tokens": T, "context": CTX, "block_ms": round(times["block"], 4),
                                  "serial_ms": round(times["serial"], 4), "single_ms": round(times["single"], 4),
                                  "block_over_single": round(times["block"] / times["single"], 3),
                                  "bit_identical": same, "api": "host buffers, synchronous (median of 10)"}
        log(f"[bench] block verify {T} tokens @{CTX}: block {times['block']:.4f} ms, "
            f"serial {times['serial']:.4f} ms, single {times['single']:.4f} ms, identical {same}")
        L.kvl_mla_compressed_q8_state_free(C.byref(bst))

    # ---- batch-1 decode, the call src/generate.c:61 makes per layer and token ---------------
    # config 0: FP32 state (KvlMlaCompressedState), 1024 rows from the state prefill of seeded
    # N(0,1) hidden states; config 1: Q8 state, 8192 rows (synthetic, generated on the device).
    # Weights: layer 0 of the stack (bound). Host API (host buffers, synchronous, median of 50),
    # device time of the same decode (stream-ordered call with KVL_MLA_NO_ADVANCE, 20 of them
    # captured in one HIP graph, replayed), the stage times (events around each launch of eager
    # device calls), and the reference C path on the same state and token.
    if not args.no_batch1:
        fp = lambda a: a.ctypes.data_as(abi.f32p)  # noqa: E731
        legs = {}
        for name, kind, ctx_len in (("c0", "f32", 1024), ("c1", "q8", 8192)):
            T = abi.KvlMlaCompressedState if kind == "f32" else abi.KvlMlaCompressedQ8State
            pre = "compressed_state" if kind == "f32" else "compressed_q8_state"
            dec = L.kvl_mla_decode_compressed_bf16 if kind == "f32" else L.kvl_mla_decode_compressed_q8_bf16
            ddev = (L.kvl_mla_decode_compressed_batch_device if kind == "f32"
                    else L.kvl_mla_decode_compressed_q8_batch_device)
            row_b = 4 * (cfg.kv_lora_rank + cfg.qk_rope_dim) if kind == "f32" else Q8_ROW
            st = T()
            lib.check(getattr(L, f"kvl_mla_{pre}_init")(C.byref(st), C.byref(cfg), ctx_len + 1), "state init")
            xs = np.ascontiguousarray(inputs.hidden(cfg, 0xC0 if kind == "f32" else 0xC1, ctx_len + 1))
            if kind == "f32":
                lib.check(L.kvl_mla_compressed_state_prefill_bf16(fp(xs[:ctx_len]), ctx_len, C.byref(cfg),
                                                                  C.byref(wstructs[0]), C.byref(st)), "state prefill")
            else:
                lib.check(L.kvl_mla_compressed_q8_state_fill_synthetic(C.byref(st), 0, ctx_len, 0xC1), "fill")
                lib.check(L.kvl_mla_compressed_q8_state_pull(C.byref(st), 0, ctx_len), "pull")
            xq = np.ascontiguousarray(xs[ctx_len])
            out = np.zeros(H, np.float32)

            def host_call():
                lib.check(dec(fp(out), fp(xq), ctx_len, C.byref(cfg), C.byref(wstructs[0]), C.byref(st)), "decode")
                lib.check(getattr(L, f"kvl_mla_{pre}_truncate")(C.byref(st), ctx_len), "truncate")
            for _ in range(5):
                host_call()
            ts = []
            for _ in range(50):
                t0_ = time.perf_counter()
                host_call()
                ts.append(time.perf_counter() - t0_)
            host_ms = float(np.median(ts)) * 1e3
            gpu_out = out.copy()
            # device time: 20 stream-ordered decodes in one graph
            arr1 = (C.POINTER(T) * 1)(C.pointer(st))
            d_i = L.kvl_mla_device_alloc(xq.nbytes)
            d_o = L.kvl_mla_device_alloc(xq.nbytes)
            lib.check(L.kvl_mla_copy_to_device(d_i, xq.ctypes.data, xq.nbytes), "h2d")
            for _ in range(3):
                lib.check(ddev(d_o, d_i, 1, C.byref(cfg), C.byref(wstructs[0]), arr1, lib.NO_ADVANCE), "device decode")
            lib.check(L.kvl_mla_synchronize(), "sync")
            lib.check(L.kvl_mla_timing_enable(1), "timing on")
            for _ in range(20):
                lib.check(ddev(d_o, d_i, 1, C.byref(cfg), C.byref(wstructs[0]), arr1, lib.NO_ADVANCE), "device decode")
            lib.check(L.kvl_mla_synchronize(), "sync")
            lib.check(L.kvl_mla_timing_read(ms, cnt), "timing read")
            lib.check(L.kvl_mla_timing_enable(0), "timing off")
            st_ms = {nm: ms[i] / cnt[i] for i, nm in enumerate(lib.STAGES) if cnt[i]}
            lib.check(L.kvl_mla_capture_begin(), "capture begin")
            rc = 0
            try:
                for _ in range(20):
                    rc = rc or ddev(d_o, d_i, 1, C.byref(cfg), C.byref(wstructs[0]), arr1, lib.NO_ADVANCE)
            finally:
                g1 = C.c_void_p()
                rc2 = L.kvl_mla_capture_end(C.byref(g1))
            lib.check(rc, "captured decode")
            lib.check(rc2, "capture end")
            lib.check(L.kvl_mla_graph_launch(g1), "graph launch")
            lib.check(L.kvl_mla_synchronize(), "sync")
            gt = []
            for _ in range(5):
                e0_ = L.kvl_mla_event_record()
                lib.check(L.kvl_mla_graph_launch(g1), "graph launch")
                e1_ = L.kvl_mla_event_record()
                lib.check(L.kvl_mla_synchronize(), "sync")
                gt.append(L.kvl_mla_event_elapsed_ms(e0_, e1_) / 20)
                L.kvl_mla_event_destroy(e0_)
                L.kvl_mla_event_destroy(e1_)
            L.kvl_mla_graph_destroy(g1)
            dev_ms = float(np.median(gt))
            L.kvl_mla_device_free(d_i)
            L.kvl_mla_device_free(d_o)
            hist_b = (ctx_len + 1) * row_b
            total_b = wb + hist_b + 2 * 4 * H
            entry = {
                "state": "FP32 (KvlMlaCompressedState)" if kind == "f32" else "Q8 (KvlMlaCompressedQ8State)",
                "context": ctx_len, "host_api_ms": round(host_ms, 4), "device_ms": round(dev_ms, 4),
                "device_gbs": round(total_b / (dev_ms * 1e-3) / 1e9, 1), "algorithmic_bytes": total_b,
                "stages_ms_per_launch": {k: round(v, 5) for k, v in st_ms.items()},
                # a lone Q8 decode runs the projection, query preparation, append, attention and
                # combine in one launch (no gemv_in stage): its stage time is not the attention's
                "attention_gbs": (round(hist_b / (st_ms["attention"] * 1e-3) / 1e9, 1) if "gemv_in" in st_ms
                                  else None),
                "attention_launch": ("the attention alone" if "gemv_in" in st_ms else
                                     "k_attn_q8_mfma<true, true, kCombCross>: q_proj | kv_a, query preparation, "
                                     "row append, attention and combine in one launch"),
                "timing": "host API: median of 50 synchronous calls; device: 20 stream-ordered calls in one HIP "
                          "graph, median of 5 replays; stages: events around each launch of eager calls"}
            if not args.no_cpu:
                import pyoracle
                from helpers import rel_err
                ref = pyoracle.load_reference("avx2")
                ckind = "reference" if ref is not None else "port"
                cpu = ref if ref is not None else pyoracle.load_oracle()
                pfx = "kvl_" if ref is not None else "orc_"
                cfn = getattr(cpu, pfx + ("mla_decode_compressed_bf16" if kind == "f32"
                                          else "mla_decode_compressed_q8_bf16"))
                co = np.zeros(H, np.float32)
                cts = []
                for _ in range(4):
                    t0_ = time.perf_counter()
                    if cfn(fp(co), fp(xq), ctx_len, C.byref(cfg), C.byref(wstructs[0]), C.byref(st)) != 0:
                        raise RuntimeError("CPU decode failed")
                    cts.append(time.perf_counter() - t0_)
                    st.len = ctx_len
                cms = float(np.median(cts[1:])) * 1e3
                entry["cpu_baseline"] = {"ms": round(cms, 3), "gbs": round(total_b / (cms * 1e-3) / 1e9, 3),
                                         "cores": omp_threads(), "kind": ckind,
                                         "sample": "the same decode, median of 3 after 1 warm-up"}
                entry["parity_vs_cpu"] = {"max_rel_err": rel_err(gpu_out, co), "tolerance": 2e-3}
            legs[name] = entry
            log(f"[bench] batch-1 {name} ({kind}, {ctx_len} rows): host API {host_ms:.4f} ms, device {dev_ms:.4f} ms "
                f"({entry['device_gbs']} GB/s), attention launch {st_ms['attention'] * 1e3:.1f} us "
                f"({entry['attention_launch']})")
            getattr(L, f"kvl_mla_{pre}_free")(C.byref(st))
        result["batch1_decode"] = legs

    # ---- causal prefill, 4096 tokens -----------------------------------------------------
    if not args.no_prefill:
        S = args.prefill_tokens
        # The 4096-token prefill workload takes bf16 inputs from seeded N(0,1) hidden states (the
        # q|kv_a GEMM's lo pass is then skipped); also timed with fp32 x, as a layer sees its
        # RMSNorm output (full mantissa: hi and lo passes)
        x32 = np.random.default_rng(0xC3).standard_normal((S, H), dtype=np.float32)
        xbf = np.ascontiguousarray(inputs.bf16_bits_to_f32(inputs.f32_to_bf16_bits(x32)))
        d_px = L.kvl_mla_device_alloc(x32.nbytes)
        d_po = L.kvl_mla_device_alloc(x32.nbytes)

        def time_prefill(xs):
            # steady state: 3 warm-up calls, then the median of 5 trials of 10 back-to-back calls
            # (a handful of calls right after the GPU idled read 5-10 % slower)
            lib.check(L.kvl_mla_copy_to_device(d_px, xs.ctypes.data, xs.nbytes), "h2d")
            for _ in range(3):
                lib.check(L.kvl_mla_prefill_device(d_po, d_px, S, C.byref(cfg), C.byref(wstructs[0])), "prefill")
            lib.check(L.kvl_mla_synchronize(), "sync")
            reps, trials = 10, []
            for _ in range(5):
                p0 = L.kvl_mla_event_record()
                for _ in range(reps):
                    lib.check(L.kvl_mla_prefill_device(d_po, d_px, S, C.byref(cfg), C.byref(wstructs[0])), "prefill")
                p1 = L.kvl_mla_event_record()
                trials.append(L.kvl_mla_event_elapsed_ms(p0, p1) / reps)
                L.kvl_mla_event_destroy(p0)
                L.kvl_mla_event_destroy(p1)
            return float(np.median(trials))

        pms_32 = time_prefill(np.ascontiguousarray(x32))
        pms = time_prefill(xbf)
        flops = prefill_flops(S, cfg)
        tf = flops / (pms * 1e-3) / 1e12
        result["prefill"] = {"tokens": S, "ms": round(pms, 4), "tflops": round(tf, 2),
                             "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4),
                             "algorithmic_gflop": round(flops / 1e9, 3), "x": "bf16 N(0,1)",
                             "fp32_x_ms": round(pms_32, 4),
                             "fp32_x_tflops": round(flops / (pms_32 * 1e-3) / 1e12, 2)}
        log(f"[bench] prefill S={S}: {pms:.3f} ms, {tf:.1f} TFLOP/s (bf16 x); {pms_32:.3f} ms with fp32 x")
        # the same prefill filling a Q8 state of the S tokens on the way (one call)
        qs = abi.KvlMlaCompressedQ8State()
        lib.check(L.kvl_mla_compressed_q8_state_init(C.byref(qs), C.byref(cfg), S), "state init")
        fms = []
        for rep in range(4):
            L.kvl_mla_compressed_q8_state_reset(C.byref(qs))
            lib.check(L.kvl_mla_synchronize(), "sync")
            f0 = L.kvl_mla_event_record()
            lib.check(L.kvl_mla_prefill_compressed_q8_state_device(d_po, d_px, S, C.byref(cfg), C.byref(wstructs[0]),
                                                                   C.byref(qs)), "prefill + state fill")
            f1 = L.kvl_mla_event_record()
            if rep:
                fms.append(L.kvl_mla_event_elapsed_ms(f0, f1))
        fm = float(np.median(fms))
        result["prefill"]["with_q8_state_fill_ms"] = round(fm, 4)
        log(f"[bench] prefill + Q8 state fill S={S}: {fm:.3f} ms")
        if not args.no_cpu:
            # the reference prefill (src/mla_prefill_streaming.c:78-206, built from its sources; the
            # oracle restatement where that build is absent) on the host cores at two lengths,
            # extrapolated to S with T(S) = a S + b S^2 (linear projections, causal attention);
            # the GPU prefill of the same tokens doubles as a parity check
            import pyoracle
            from helpers import rel_err
            ref = pyoracle.load_reference("avx2")
            pkind = "reference" if ref is not None else "port"
            pfn = ref.kvl_mla_prefill_bf16 if ref is not None else pyoracle.load_oracle().orc_mla_prefill_streaming
            samples, perr = {}, []
            for Sc in (S // 4, S // 2):
                xc = np.ascontiguousarray(xbf[:Sc])
                oc = np.zeros((Sc, H), np.float32)
                og = np.zeros((Sc, H), np.float32)
                ts = time.perf_counter()
                if pfn(oc.ctypes.data_as(abi.f32p), xc.ctypes.data_as(abi.f32p), Sc, C.byref(cfg),
                       C.byref(wstructs[0])) != 0:
                    raise RuntimeError("CPU prefill failed")
                samples[Sc] = time.perf_counter() - ts
                lib.check(L.kvl_mla_prefill_bf16(og.ctypes.data_as(abi.f32p), xc.ctypes.data_as(abi.f32p), Sc,
                                                 C.byref(cfg), C.byref(wstructs[0])), "prefill parity")
                perr.append(rel_err(og, oc))
            (s1, t1), (s2, t2) = sorted(samples.items())
            bq = max(0.0, (t2 * s1 - t1 * s2) / (s1 * s2 * (s2 - s1)))
            aq = (t1 - bq * s1 * s1) / s1 if bq > 0 else t2 / s2
            tS = aq * S + bq * S * S
            result["prefill"]["cpu_baseline"] = {
                "value": round(flops / tS / 1e12, 4), "unit": "TFLOP/s", "cores": omp_threads(), "kind": pkind,
                "sample": f"S={s1} ({t1:.2f} s) and S={s2} ({t2:.2f} s) measured on the same tokens and weights; "
                          f"S={S} extrapolated with T = aS + bS^2 ({tS:.1f} s)"}
            result["prefill"]["parity_vs_cpu"] = {"max_rel_err": float(max(perr)), "tokens": [s1, s2],
                                                  "tolerance": 2e-3}
            log(f"[bench] prefill CPU baseline ({pkind}): S={s1} {t1:.2f} s, S={s2} {t2:.2f} s -> S={S} "
                f"{tS:.1f} s; GPU vs CPU {max(perr):.2e}")
        L.kvl_mla_compressed_q8_state_free(C.byref(qs))
        L.kvl_mla_device_free(d_px)
        L.kvl_mla_device_free(d_po)

    # ---- 64 ragged sequences, one decode token each: the BF16-latent state (1152 B/row), and
    # the FP32 state of the same bf16-valued rows (2304 B/row) beside it -------------------------
    if not args.no_ragged:
        rng = np.random.default_rng(0xC8)
        lens = rng.integers(512, 32769, size=64)
        RB = len(lens)
        xr = np.ascontiguousarray(inputs.hidden(cfg, 0xC8, RB, tag="query"))
        d_rx = L.kvl_mla_device_alloc(xr.nbytes)
        d_ro = L.kvl_mla_device_alloc(xr.nbytes)
        lib.check(L.kvl_mla_copy_to_device(d_rx, xr.ctypes.data, xr.nbytes), "h2d")
        kinds = {
            "bf16": (abi.KvlMlaCompressedBF16State, "compressed_bf16_state", 2,
                     L.kvl_mla_decode_compressed_bf16_batch_device, "bf16 rows (1152 B/row)"),
            "f32": (abi.KvlMlaCompressedState, "compressed_state", 4,
                    L.kvl_mla_decode_compressed_batch_device, "fp32 rows (2304 B/row) of the same bf16 values"),
        }
        for kind, (T, name, eb, rdec, what) in kinds.items():
            rstates = []
            for i, n in enumerate(lens):
                st = T()
                lib.check(getattr(L, f"kvl_mla_{name}_init")(C.byref(st), C.byref(cfg), int(n) + 1), "ragged init")
                lib.check(getattr(L, f"kvl_mla_{name}_fill_synthetic")(C.byref(st), 0, int(n), 0xC80 + i),
                          "ragged fill")
                rstates.append(st)
            rarr = (C.POINTER(T) * RB)(*[C.pointer(s) for s in rstates])
            for _ in range(3):
                lib.check(rdec(d_ro, d_rx, RB, C.byref(cfg), C.byref(wstructs[0]), rarr, lib.NO_ADVANCE), "ragged")
            lib.check(L.kvl_mla_synchronize(), "sync")
            reps = 10
            r0 = L.kvl_mla_event_record()
            for _ in range(reps):
                lib.check(rdec(d_ro, d_rx, RB, C.byref(cfg), C.byref(wstructs[0]), rarr, lib.NO_ADVANCE), "ragged")
            r1 = L.kvl_mla_event_record()
            rms = L.kvl_mla_event_elapsed_ms(r0, r1) / reps
            L.kvl_mla_event_destroy(r0)
            L.kvl_mla_event_destroy(r1)
            rbytes = wb + int((lens + 1).sum()) * eb * (cfg.kv_lora_rank + cfg.qk_rope_dim)
            rgbs = rbytes / (rms * 1e-3) / 1e9
            entry = {
                "sequences": RB, "rows": int(lens.sum()), "context": "uniform 512..32768 (seeded)",
                "state": what, "ms": round(rms, 4), "gbs": round(rgbs, 1),
                "frac_hbm_peak": round(rgbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": rbytes,
                "api": "device buffers, stream-ordered, eager launches"}
            result["ragged_decode" if kind == "bf16" else "ragged_decode_fp32_state"] = entry
            log(f"[bench] ragged 64 sequences ({int(lens.sum())} rows, {kind} state): {rms:.4f} ms, {rgbs:.1f} GB/s")
            for st in rstates:
                getattr(L, f"kvl_mla_{name}_free")(C.byref(st))
        L.kvl_mla_device_free(d_rx)
        L.kvl_mla_device_free(d_ro)

    # ---- measured memory peak: a plain 16-byte copy kernel over 1 GiB (read + write) -------
    if not args.no_peak:
        nb = 1 << 30
        pa = L.kvl_mla_device_alloc(nb)
        pb = L.kvl_mla_device_alloc(nb)
        if pa and pb:
            for _ in range(3):
                lib.check(L.kvl_mla_copy_kernel(pb, pa, nb), "copy")
            lib.check(L.kvl_mla_synchronize(), "sync")
            c0 = L.kvl_mla_event_record()
            for _ in range(5):
                lib.check(L.kvl_mla_copy_kernel(pb, pa, nb), "copy")
            c1 = L.kvl_mla_event_record()
            cms = L.kvl_mla_event_elapsed_ms(c0, c1) / 5
            peak = 2 * nb / (cms * 1e-3) / 1e9
            for _ in range(3):
                lib.check(L.kvl_mla_read_kernel(pa, nb), "read")
            lib.check(L.kvl_mla_synchronize(), "sync")
            c2 = L.kvl_mla_event_record()
            for _ in range(5):
                lib.check(L.kvl_mla_read_kernel(pa, nb), "read")
            c3 = L.kvl_mla_event_record()
            rms_ = L.kvl_mla_event_elapsed_ms(c2, c3) / 5
            rpeak = nb / (rms_ * 1e-3) / 1e9
            for e in (c0, c1, c2, c3):
                L.kvl_mla_event_destroy(e)
            result["measured_peak"] = {"read_gbs": round(rpeak, 1), "copy_gbs_read_plus_write": round(peak, 1),
                                       "bytes": nb, "nominal_gbs": HBM_PEAK_GBS,
                                       "attention_frac_of_measured_read": round(roofline["achieved"] / rpeak, 4)}
            roofline["measured_read_peak"] = round(rpeak, 1)
            log(f"[bench] measured bandwidth: streaming read {rpeak:.1f} GB/s, copy {peak:.1f} GB/s (read + write)")
            # the fixed cost of a kernel boundary in a HIP graph: 100 empty kernels back to back
            if not args.eager:
                lib.check(L.kvl_mla_capture_begin(), "capture begin")
                try:
                    for _ in range(100):
                        lib.check(L.kvl_mla_empty_kernel(), "empty kernel")
                finally:
                    ge = C.c_void_p()
                    rc = L.kvl_mla_capture_end(C.byref(ge))
                lib.check(rc, "capture end")
                lib.check(L.kvl_mla_graph_launch(ge), "graph launch")
                lib.check(L.kvl_mla_synchronize(), "sync")
                c4 = L.kvl_mla_event_record()
                for _ in range(5):
                    lib.check(L.kvl_mla_graph_launch(ge), "graph launch")
                c5 = L.kvl_mla_event_record()
                floor_us = L.kvl_mla_event_elapsed_ms(c4, c5) / 500 * 1e3
                for e in (c4, c5):
                    L.kvl_mla_event_destroy(e)
                L.kvl_mla_graph_destroy(ge)
                result["measured_peak"]["kernel_boundary_us"] = round(floor_us, 3)
                log(f"[bench] kernel boundary in a HIP graph (empty 256 x 1024 kernels): {floor_us:.2f} us")
        for q in (pa, pb):
            if q:
                L.kvl_mla_device_free(q)

    if args.calibrate_copy:
        nb = args.calibrate_copy << 20
        a = L.kvl_mla_device_alloc(nb)
        b = L.kvl_mla_device_alloc(nb)
        for _ in range(3):
            lib.check(L.kvl_mla_copy_kernel(b, a, nb), "copy")
        lib.check(L.kvl_mla_synchronize(), "sync")
        c0 = L.kvl_mla_event_record()
        lib.check(L.kvl_mla_copy_kernel(b, a, nb), "copy")
        c1 = L.kvl_mla_event_record()
        cms = L.kvl_mla_event_elapsed_ms(c0, c1)
        result["copy_calibration"] = {"bytes_each_way": nb, "ms": round(cms, 4),
                                      "gbs_read_plus_write": round(2 * nb / (cms * 1e-3) / 1e9, 1)}
        L.kvl_mla_device_free(a)
        L.kvl_mla_device_free(b)

    if graph is not None:
        L.kvl_mla_graph_destroy(graph)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
