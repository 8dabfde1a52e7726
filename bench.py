#!/usr/bin/env python3
"""Benchmark of the quantized embedding-inference hot path on one MI355X.

Workload (benchmark config c2, the config the headline metric is quoted on):
TurboQuant flat retrieval scoring -- 1,000,000 vectors x 384 dims, 4-bit codes
+ one f32 norm each (196 B/vector), seeded rotation, 64 unit queries, top-100.
A step is one full top-k call (prepare, sample threshold, filtered scan,
finalize) over the device-resident corpus with device-resident queries.

Prints one JSON line (the driver's contract), with `roofline` for the
dominant kernel (the filtered scan, timed per launch with HIP events that its
own dispatches record, against 8 TB/s and against a copy kernel's measured
rate) and `cpu_baseline` (the C oracle's reference-loop port on a bounded
sample, single-threaded and all-core). The other benchmark configs ride on the
same line as sub-objects, each with its own roofline and CPU baseline:
`tiny_c1` (tiny embed, µs per call), `two_stage_c2` (TurboQuant top-200 +
f16 rerank top-100), `maxsim_c5` (MaxSim over 100k documents of 128 vectors,
against the int8 MFMA peak), `encoder_c3` / `encoder_c4` (q8 BERT-style
encoder forward, tokens/s, with a per-stage breakdown). `mfma_ceiling` is the
rate and shader clock a stream of independent MFMAs reaches on zero and on
full-range random operands; the MFMA-bound legs carry their fraction of that
clock-limited ceiling beside their fraction of the published peak.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "q8 encoder tokens/s @seq512; TurboQuant vectors scored/s; % of roofline"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "tq_scan_filter_c2_traffic.json")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _cpu_threads() -> int:
    """Host threads for the all-core CPU variants: the job's CPU share
    (OMP_NUM_THREADS, 16 on the GPU box), else every core."""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "") or os.cpu_count() or 1))
    except ValueError:
        return os.cpu_count() or 1


def _threaded(fn, chunks, threads: int) -> float:
    """Runs fn over chunks on `threads` host threads (the oracle's ctypes calls
    release the GIL); returns the wall seconds."""
    from concurrent.futures import ThreadPoolExecutor
    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(fn, chunks))
    return time.perf_counter() - t0


def cpu_baseline(corpus, queries, nq_sample: int) -> dict:
    import oracle  # the checker/baseline only; never the measured path
    q = queries[:nq_sample]
    args = (corpus.rotation, corpus.dim, corpus.bits, corpus.codebook, corpus.codebook_scale,
            corpus.codes, corpus.norms, 100)
    t0 = time.perf_counter()
    oracle.tq_topk(q, *args)
    dt = time.perf_counter() - t0
    # All-core variant: queries split over the host threads.
    threads = _cpu_threads()
    nq_all = max(threads * 4, nq_sample)
    qa = np.concatenate([queries] * (-(-nq_all // len(queries))))[:nq_all]
    chunks = np.array_split(qa, threads)
    dt_all = _threaded(lambda c: oracle.tq_topk(c, *args), chunks, threads)
    return {
        "value": nq_sample * corpus.n / dt,
        "unit": "vectors scored/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{nq_sample} queries x {corpus.n} vectors, top-100 ({dt:.2f} s): single-threaded C "
                  "restatement of the loop of topTurboQuantRetrievalScoresWithStats (score every "
                  "vector, size-k heap, final sort) scoring with this build's exact integer "
                  "estimator (int16 query x int8-grid codebook through a byte LUT), not the "
                  "reference module's f32 estimator",
        "all_core": {"value": nq_all * corpus.n / dt_all, "cores": threads,
                     "sample": f"{nq_all} queries split over {threads} threads ({dt_all:.2f} s)"},
        "cpu_model": _cpu_model(),
        "host_cores": os.cpu_count(),
    }


ENCODER_CONFIGS = {
    # name: layers, hidden, heads, ffn, batch, seq, len_lo, len_hi, weight seed, ids seed, len seed
    "c3": (6, 384, 12, 1536, 64, 512, 32, 512, 7, 8, 9),
    "c4": (4, 512, 8, 2048, 4, 8192, 4096, 8192, 10, 11, 10),
}


def encoder_cpu_baseline(w, ids, mask, lens, name: str) -> dict:
    """The oracle's restatement of BERTEncoderLayerReference
    (bert_encoder_layer_ops.go:80-495: f64 dense over every padded row,
    per-(query, head) f64 attention over active keys), OpenMP over rows and
    query heads like the reference's goroutines, timed on a sample and
    extrapolated to the whole batch with its work model: per sequence and
    layer, T rows x (4 H^2 + 2 H F) dense MAC + 2 T len H attention MAC."""
    import oracle
    B, T = ids.shape
    H, F, L = w.hidden, w.intermediate, len(w.layers)
    if name == "c3":
        nseq, nlay = 16, L              # 16 whole sequences, every layer
    else:
        nseq, nlay = 1, 1               # c4: one sequence through one layer
    layers = [Ly.dequantized() for Ly in w.layers[:nlay]]

    def work(blens, nl):
        return float(sum(nl * T * (4 * H * H + 2 * H * F) + 2.0 * nl * T * int(n) * H
                         for n in blens))

    t0 = time.perf_counter()
    oracle.bert_embed(w.tok, w.pos, w.typ, w.emb_gamma, w.emb_beta, layers, ids[:nseq],
                      mask[:nseq], None, w.heads, w.ln_eps)
    dt = time.perf_counter() - t0
    full_s = dt * work(lens, L) / work(lens[:nseq], nlay)
    threads = _cpu_threads()
    return {
        "value": B * T / full_s,
        "unit": f"tokens/s (batch x {T} per forward)",
        "valid_tokens_per_s": float(lens.sum()) / full_s,
        "cores": threads,
        "kind": "port",
        "sample": (f"{nseq} of {B} sequences through {nlay} of {L} layers in {dt:.2f} s "
                   f"(f64 C restatement of BERTEncoderLayerReference, OpenMP on {threads} "
                   f"threads), extrapolated by the dense + attention MAC count to the whole "
                   f"batch: {full_s:.1f} s per forward"),
        "cpu_model": _cpu_model(),
    }


def encoder_leg(rt, steps: int, name: str = "c3", cpu: bool = True) -> dict:
    """Benchmark config c3 (q8 BERT-style encoder, 6 layers, hidden 384, 12
    heads, FFN 1536, batch 64 x seq 512, lengths U[32, 512]) or config 4 (long
    context: 4 layers, hidden 512, 8 heads, FFN 2048, batch 4 x 8192, lengths
    U[4096, 8192]); inputs resident on device."""
    from eos_amd import datagen
    from eos_amd.encoder import Encoder
    from eos_amd.runtime import DeviceBuffer

    L, H, NH, F, B, T, lo, hi, sw, si, sl = ENCODER_CONFIGS[name]
    w = datagen.bert_q8_weights(L, H, NH, F, 30522, T, seed=sw)
    ids, mask, lens = datagen.encoder_batch(B, T, 30522, lo, hi, si, sl)
    enc = Encoder(rt, w)
    d_ids = DeviceBuffer.from_array(rt, ids)
    d_mask = DeviceBuffer.from_array(rt, mask)
    d_out = DeviceBuffer(rt, B * H * 4)
    for _ in range(2):
        enc.embed_device(d_ids, d_mask, B, T, d_out)
    rt.sync()
    rt.mark(2)
    for _ in range(steps):
        enc.embed_device(d_ids, d_mask, B, T, d_out)
    rt.mark(3)
    ms = rt.elapsed_ms(2, 3) / steps
    # Per-kernel breakdown from a separate pass with every launch bracketed.
    rt.profile_reset()
    rt.profile_select(None)
    rt.profile(True)
    for _ in range(steps):
        enc.embed_device(d_ids, d_mask, B, T, d_out)
    rt.sync()
    kernels = {}
    for kname in ("eos_enc_pack", "eos_enc_embed", "enc_gemm_qkv", "eos_enc_attn", "enc_tail",
                  "enc_gemm_o", "enc_ln", "enc_gemm_ffn_up", "enc_gemm_ffn_down", "eos_enc_pool"):
        n, t = rt.profile_read(kname)
        kernels[kname] = t / steps
    rt.profile(False)
    valid = int(lens.sum())
    lin = 2.0 * valid * L * (3 * H * H + H * H + 2 * H * F)
    att = 2.0 * 2.0 * float(np.sum(lens.astype(np.float64) ** 2)) * H * L
    flops = lin + att
    achieved = flops / (ms / 1e3) / 1e12
    enc.release()
    base = None
    if cpu:
        log(f"encoder {name}: cpu baseline")
        base = encoder_cpu_baseline(w, ids, mask, lens, name)
    return {
        "metric": f"q8 encoder tokens/s @seq{T}",
        "value": B * T / (ms / 1e3),
        "unit": f"tokens/s (batch x {T} per forward)",
        "valid_tokens_per_s": valid / (ms / 1e3),
        "ms_per_forward": ms,
        "config": {"layers": L, "hidden": H, "heads": NH, "ffn": F, "batch": B, "seq": T,
                   "valid_tokens": valid},
        "dtype": ("QKV and FFN-up: int8 activations (per-row scales) x int8 weights "
                  "(per-channel scales) on int8 MFMA, exact i32; O, FFN-down: f16 activations x "
                  "int8 weight codes on f16 MFMA, f32 accumulate; attention f16 MFMA, f32 softmax"),
        "roofline": {"bound": "mfma", "achieved": achieved, "unit": "TFLOP/s",
                     "peak_f16": 2500.0, "frac_f16": achieved / 2500.0,
                     "peak_int8": 5000.0, "frac_int8": achieved / 5000.0,
                     "flops_per_forward_valid": flops,
                     "int8_share_of_gemm_flops": (3 * H * H + H * F) / (4 * H * H + 2 * H * F),
                     "int8_share_of_flops": 2.0 * valid * L * (3 * H * H + H * F) / flops},
        "breakdown_ms": kernels,
        "cpu_baseline": base,
    }


def tq_shard_leg(rt, n: int, queries: int, k: int, steps: int, warmup: int) -> dict:
    """The c2 scan at one GPU's shard of an 8-GPU job (N / 8 vectors: the
    corpus rows are the unit a multi-GPU run would split): one stream, the
    same top-k pipeline, and the filter scan's per-launch time."""
    from eos_amd import datagen
    from eos_amd.runtime import DeviceBuffer
    from eos_amd.turboquant import TurboQuantIndex

    corpus = datagen.baseline_flat_corpus(n=n)
    q = datagen.baseline_queries(queries, corpus.dim)
    idx = TurboQuantIndex(rt, corpus.codes, corpus.norms, corpus.dim, corpus.bits, corpus.codebook,
                          corpus.codebook_scale, corpus.rotation)
    kk = idx.effective_k(k)
    dq = DeviceBuffer.from_array(rt, q)
    dids = DeviceBuffer(rt, queries * kk * 8)
    dsc = DeviceBuffer(rt, queries * kk * 4)
    # top_k_device: the exact fallback is gated on the device, so every
    # timed step is final without a host round trip.
    for _ in range(warmup):
        idx.top_k_device(dq, queries, k, dids, dsc, with_stats=False)
    rt.sync()
    rt.mark(4)
    for _ in range(steps):
        idx.top_k_device(dq, queries, k, dids, dsc, with_stats=False)
    rt.mark(5)
    ms = rt.elapsed_ms(4, 5) / steps
    rt.profile_reset()
    rt.profile_select("tq_scan_filter")
    rt.profile(True)
    for _ in range(steps):
        idx.top_k_device(dq, queries, k, dids, dsc, with_stats=False)
    rt.sync()
    nf, msf = rt.profile_read("tq_scan_filter")
    rt.profile(False)
    avg = msf / max(nf, 1)
    bytes_per_launch = n * (corpus.dim * corpus.bits // 8 + 4)
    for b in (dq, dids, dsc):
        b.free()
    idx.release()
    return {
        "metric": "TurboQuant vectors scored/s (one GPU's shard of an 8-GPU job)",
        "value": queries * n / (ms / 1e3), "unit": "vectors scored/s", "ms_per_batch": ms,
        "config": {"workload": "turboquant_flat_c2_shard8", "n": n, "dim": corpus.dim,
                   "bits": corpus.bits, "queries": queries, "k": k, "streams": 1},
        "roofline": {"bound": "hbm", "kernel": "tq_scan_filter", "avg_launch_ms": avg,
                     "bytes_per_launch": bytes_per_launch,
                     "achieved": bytes_per_launch / (avg / 1e3) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": bytes_per_launch / (avg / 1e3) / 1e9 / HBM_PEAK_GBS},
    }


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def tq_leg(rt, args) -> dict:
    """Benchmark config c2 (the bench line's workload)."""
    from eos_amd import datagen
    from eos_amd.runtime import DeviceBuffer, Runtime
    from eos_amd.turboquant import TurboQuantIndex

    log("generating corpus")
    corpus = datagen.baseline_flat_corpus(n=args.n)
    queries = datagen.baseline_queries(args.queries, corpus.dim)
    idx = TurboQuantIndex(rt, corpus.codes, corpus.norms, corpus.dim, corpus.bits, corpus.codebook,
                          corpus.codebook_scale, corpus.rotation)
    kk = idx.effective_k(args.k)
    dq = DeviceBuffer.from_array(rt, queries)
    dids = DeviceBuffer(rt, args.queries * kk * 8)
    dsc = DeviceBuffer(rt, args.queries * kk * 4)
    # One status row per step: the deferred path leaves each step's exactness
    # flags on the device; the timed region checks them all once at its end
    # and repairs any flagged step before the clock stops.
    dstat = DeviceBuffer(rt, max(args.steps, args.warmup, 1) * args.queries * 4)
    srow = args.queries * 4
    log(f"warmup {args.warmup}")
    for i in range(args.warmup):
        idx.top_k_device_deferred(dq, args.queries, args.k, dids, dsc, dstat.view(i * srow, srow))
    rt.sync()
    views = [dstat.view(i * srow, srow) for i in range(args.steps)]

    def timed(handles, outs):
        """K steps, step i on handle i % len(handles) (its own stream and
        output buffers), bracketed by events on the first runtime, which waits
        for the others before its closing event. Flagged steps are repaired
        inside the region. Returns (ms, enqueue_ms, wall_ms, repaired)."""
        for h in handles:
            h.rt.sync()
        gc.disable()
        t0 = time.perf_counter()
        rt.mark(0)
        for h in handles[1:]:
            h.rt.wait_for(rt)
        for i in range(args.steps):
            j = i % len(handles)
            handles[j].top_k_device_deferred(dq, args.queries, args.k, outs[j][0], outs[j][1], views[i])
        enqueue_ms = (time.perf_counter() - t0) * 1e3
        for h in handles[1:]:
            rt.wait_for(h.rt)
        flags = dstat.download(np.int32, (args.steps, args.queries))  # waits for rt's stream
        repaired = int(np.count_nonzero(np.any(flags != 0, axis=1)))
        for i in np.nonzero(np.any(flags != 0, axis=1))[0]:
            idx.repair_device(dq, args.queries, args.k, dids, dsc, dstat.view(int(i) * srow, srow))
        rt.mark(1)
        ms = rt.elapsed_ms(0, 1)
        wall_ms = (time.perf_counter() - t0) * 1e3
        gc.enable()
        return ms, enqueue_ms, wall_ms, repaired

    # Timed regions: every launch runs bare (an event pair around a launch
    # costs ~5 us of stream time on each side). The one-stream region gives the
    # latency of a batch; with several streams, consecutive batches rotate
    # over handles on the same resident corpus and overlap on the GPU.
    log(f"timing {args.steps} steps on one stream")
    lat_ms, _, _, _ = timed([idx], [(dids, dsc)])
    handles, outs = [idx], [(dids, dsc)]
    for _ in range(1, args.streams):
        rt_s = Runtime(0)
        h = idx.share(rt_s)
        outs.append((DeviceBuffer(rt_s, args.queries * kk * 8), DeviceBuffer(rt_s, args.queries * kk * 4)))
        handles.append(h)
        for i in range(args.warmup):
            h.top_k_device_deferred(dq, args.queries, args.k, outs[-1][0], outs[-1][1], views[0])
    if args.streams > 1:
        log(f"timing {args.steps} steps on {args.streams} streams")
    total_ms, enqueue_ms, wall_ms, repaired = timed(handles, outs)
    # Roofline: the same steps again (one stream) with HIP events on the filter
    # scan's launches, recorded by each dispatch at the kernel's start and end
    # (hipExtModuleLaunchKernel); their average is the figure.
    rt.profile_reset()
    rt.profile_select("tq_scan_filter")
    rt.profile(True)
    for i in range(args.steps):
        idx.top_k_device_deferred(dq, args.queries, args.k, dids, dsc, dstat.view(i * srow, srow))
    rt.sync()
    n_filter, ms_filter = rt.profile_read("tq_scan_filter")
    filter_samples = rt.profile_samples("tq_scan_filter")
    rt.profile(False)
    # Per-kernel breakdown from a separate pass with every launch bracketed.
    rt.profile_reset()
    rt.profile_select(None)
    rt.profile(True)
    for i in range(args.steps):
        idx.top_k_device_deferred(dq, args.queries, args.k, dids, dsc, dstat.view(i * srow, srow))
    rt.sync()
    breakdown = {}
    for name in ("eos_tq_rotate", "eos_tq_quantize", "tq_scan_sample", "eos_tq_threshold",
                 "tq_scan_filter", "tq_rescore", "eos_tq_finalize", "tq_scan_dense",
                 "tq_fallback_select"):
        breakdown[name] = rt.profile_read(name)[1] / args.steps
    rt.profile(False)
    st = idx.top_k_device(dq, args.queries, args.k, dids, dsc, with_stats=True)
    ms_per_step = total_ms / args.steps
    for h, o in zip(handles[1:], outs[1:]):
        for b in o:
            b.free()
        h.release()
        h.rt.close()
    bytes_per_launch = corpus.n * (corpus.dim * corpus.bits // 8 + 4)
    avg_filter_ms = ms_filter / max(n_filter, 1)
    med_filter_ms = float(np.median(filter_samples)) if len(filter_samples) else avg_filter_ms
    achieved = bytes_per_launch / (med_filter_ms / 1e3) / 1e9
    traffic, traffic_note = traffic_figure()
    out = {
        "value": args.queries * corpus.n / (ms_per_step / 1e3),
        "ms_per_step": ms_per_step,
        "ms_per_batch_one_stream": lat_ms / args.steps,
        "config": {"workload": "turboquant_flat_c2", "n": corpus.n, "dim": corpus.dim,
                   "bits": corpus.bits, "queries": args.queries, "k": args.k,
                   "batches_in_flight": args.streams, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": traffic_note,
                     "kernel": "tq_scan_filter", "median_launch_ms": med_filter_ms,
                     "avg_launch_ms": avg_filter_ms, "launches_timed": int(n_filter),
                     "min_launch_ms": float(np.min(filter_samples)) if len(filter_samples) else None,
                     "bytes_per_launch": bytes_per_launch},
        "breakdown_ms_per_step": breakdown,
        "fallback_queries": st.fallback_queries,
        "repaired_steps": repaired,
        "host_wall_ms_per_step": wall_ms / args.steps,
        "host_enqueue_ms_per_step": enqueue_ms / args.steps,
        "candidates_kept_per_query": st.candidates_kept / args.queries,
    }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(corpus, queries, args.cpu_sample_queries)
    else:
        out["cpu_baseline"] = None
    idx.release()
    return out


def maxsim_leg(rt, steps: int, cpu: bool = True) -> dict:
    """Benchmark config c5: 100,000 documents x 128 token vectors of dim 128,
    2-bit codes, lognormal(0, 0.25) norms, seeded rotation; 32 queries x 32
    unit Gaussian tokens; MaxSim top-100 documents per query."""
    from eos_amd import datagen
    from eos_amd.runtime import DeviceBuffer
    from eos_amd.turboquant import TurboQuantIndex, TurboQuantMultiVectorIndex

    ndocs, doc_len, dim, bits, nq, tokens, k = 100_000, 128, 128, 2, 32, 32, 100
    log("maxsim c5: generating corpus")
    corpus = datagen.TurboQuantCorpus(ndocs * doc_len, dim, bits, 21, 22, 23)
    q = datagen.baseline_queries(nq * tokens, dim, 24).reshape(nq, tokens, dim)
    idx = TurboQuantIndex(rt, corpus.codes, corpus.norms, dim, bits, corpus.codebook,
                          corpus.codebook_scale, corpus.rotation)
    mv = TurboQuantMultiVectorIndex(idx, doc_len)
    dq = DeviceBuffer.from_array(rt, q)
    dids = DeviceBuffer(rt, nq * k * 8)
    dsc = DeviceBuffer(rt, nq * k * 4)
    mv.top_k_device(dq, nq, tokens, k, dids, dsc)
    rt.sync()
    rt.mark(6)
    for _ in range(steps):
        mv.top_k_device(dq, nq, tokens, k, dids, dsc)
    rt.mark(7)
    ms = rt.elapsed_ms(6, 7) / steps
    # Per-launch times (dispatch-recorded events) of the pipeline's kernels:
    # the sampled exact scores and threshold, the high-half bound filter (one
    # launch streams the whole corpus once for every query of the batch),
    # the exact rescoring of the listed documents, the top-k, and the gated
    # exhaustive fallback (returns at once when no query is flagged).
    labels = ("tq_maxsim_sample", "tq_maxsim_threshold", "tq_maxsim_filter", "tq_maxsim_rescore",
              "tq_maxsim_finalize", "tq_maxsim_fallback", "tq_maxsim_fallback_select")
    rt.profile_reset()
    rt.profile_select(None)
    rt.profile(True)
    reps = 3
    for _ in range(reps):
        mv.top_k_device(dq, nq, tokens, k, dids, dsc)
    rt.sync()
    breakdown = {}
    for name in labels:
        breakdown[name] = rt.profile_read(name)[1] / reps
    n_f, _ = rt.profile_read("tq_maxsim_filter")
    filt = rt.profile_samples("tq_maxsim_filter")
    rt.profile(False)
    med = float(np.median(filt)) if len(filt) else 0.0
    # The launch runs the batch's passes (4 queries each) side by side, each
    # streaming the corpus (460.8 MB, more than the 256 MB Infinity Cache).
    passes = (nq + 3) // 4
    bytes_per_launch = passes * corpus.n * (dim * bits // 8 + 4)
    hbm_gbs = bytes_per_launch / (med / 1e3) / 1e9
    # The filter multiplies the high int8 half of every int16 query token
    # against every vector: 2 x MAC per (token, vector, dim) = 3.4 T int8 ops
    # per batch in one launch. Exact scoring of every pair (both halves) is
    # twice that: the batch's algorithmic work, reported against the whole
    # pipeline's time.
    ops_filter = 2.0 * nq * tokens * corpus.n * dim
    achieved = ops_filter / (med / 1e3) / 1e12
    ops_exact = 2.0 * ops_filter
    out = {
        "metric": "MaxSim query-document pairs scored/s",
        "value": nq * ndocs / (ms / 1e3),
        "unit": "query-document pairs/s",
        "ms_per_batch": ms,
        "config": {"workload": "turboquant_maxsim_c5", "docs": ndocs, "doc_len": doc_len,
                   "dim": dim, "bits": bits, "queries": nq, "tokens": tokens, "k": k},
        "token_vector_pairs_per_s": nq * tokens * corpus.n / (ms / 1e3),
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": INT8_PEAK_TOPS,
                     "unit": "TOP/s (int8)", "frac": achieved / INT8_PEAK_TOPS,
                     "kernel": "tq_maxsim_filter", "median_launch_ms": med,
                     "launches_per_batch": n_f / reps, "int8_ops_per_launch": ops_filter,
                     "bytes_per_launch": bytes_per_launch, "hbm_gbs": hbm_gbs,
                     "hbm_frac": hbm_gbs / HBM_PEAK_GBS,
                     "exact_int8_ops_per_batch": ops_exact,
                     "exact_equivalent_tops": ops_exact / (ms / 1e3) / 1e12,
                     "exact_equivalent_frac": ops_exact / (ms / 1e3) / 1e12 / INT8_PEAK_TOPS},
        "breakdown_ms": breakdown,
    }
    if cpu:
        out["cpu_baseline"] = maxsim_cpu_baseline(corpus, q, doc_len, ndocs)
    for b in (dq, dids, dsc):
        b.free()
    idx.release()
    return out


def maxsim_cpu_baseline(corpus, q, doc_len: int, ndocs: int) -> dict:
    """The oracle's MaxSim (per query token the reference child-max over a
    document's vectors, summed over tokens) on the first 2000 documents:
    4 queries single-threaded, and all 32 queries over the host threads."""
    import oracle
    nd = 2000
    rows = nd * doc_len
    args = (corpus.rotation, corpus.dim, corpus.bits, corpus.codebook, corpus.codebook_scale,
            corpus.codes[:rows], corpus.norms[:rows], doc_len)
    t0 = time.perf_counter()
    oracle.tq_maxsim_scores(q[:4], *args)
    dt = time.perf_counter() - t0
    threads = _cpu_threads()
    chunks = [c for c in np.array_split(q, threads) if len(c)]
    dt_all = _threaded(lambda c: oracle.tq_maxsim_scores(c, *args), chunks, threads)
    return {
        "value": 4 * nd / dt,
        "unit": "query-document pairs/s",
        "cores": 1,
        "kind": "port",
        "sample": f"4 queries x {q.shape[1]} tokens against the first {nd} of {ndocs} documents "
                  f"({dt:.2f} s, single-threaded C restatement of the child-max loop, "
                  "retrieval_multivector_turboquant.go:746-808, summed over query tokens)",
        "all_core": {"value": q.shape[0] * nd / dt_all, "cores": threads,
                     "sample": f"{q.shape[0]} queries split over {threads} threads ({dt_all:.2f} s)"},
        "cpu_model": _cpu_model(),
    }


def code_object_sha256(stem: str = "tq") -> str | None:
    """SHA-256 of a built code object (eos_amd/_build/<stem>.hsaco), the
    identity of the kernels a counter file was captured on."""
    import hashlib
    from eos_amd.build import BUILD_DIR
    path = os.path.join(BUILD_DIR, f"{stem}.hsaco")
    if not os.path.exists(path):
        return None
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def traffic_figure() -> tuple:
    """HBM bytes per filter-scan launch from the committed counter summary,
    only when it was captured on the code object this run loads (else None,
    with the reason)."""
    if not os.path.exists(TRAFFIC_FILE):
        return None, "no counter summary"
    try:
        rec = json.load(open(TRAFFIC_FILE))
    except (OSError, ValueError) as e:
        return None, f"counter summary unreadable: {e}"
    want = rec.get("code_object_sha256")
    have = code_object_sha256("tq")
    if want is None or have is None or want != have:
        return None, (f"stale: counters captured on tq.hsaco {str(want)[:12]}, "
                      f"this run loads {str(have)[:12]}")
    return rec.get("hbm_bytes_per_launch"), (f"{os.path.relpath(TRAFFIC_FILE, ROOT)} "
                                             f"(tq.hsaco {have[:12]}, commit {rec.get('commit')})")


def read_calibration(rt, mb: int, reps: int = 5) -> dict:
    """A read-only stream over `mb` MB (probe kernel eos_probe_read_stream:
    16-byte non-temporal loads, 8 in flight per thread, XOR-folded into one
    word per thread): the achievable rate of a kernel that only reads, which
    is what the corpus scans are (>= 99.7 % of their bytes are reads)."""
    import ctypes as C
    from eos_amd import _lib
    from eos_amd.build import PROBE_PATH
    from eos_amd.runtime import DeviceBuffer

    img = open(PROBE_PATH, "rb").read()
    mod = C.c_void_p()
    _lib.call("eoship_module_load", rt.handle, img, C.c_size_t(len(img)), C.byref(mod))
    fn = C.c_void_p()
    _lib.call("eoship_function", mod, b"eos_probe_read_stream", C.byref(fn))
    nbytes = mb * 1_000_000 // 16 * 16
    blocks = rt.info()["compute_units"] * 8

    class Args(C.Structure):
        _fields_ = [("src", C.c_void_p), ("sink", C.c_void_p), ("words", C.c_longlong)]

    src = DeviceBuffer(rt, nbytes)
    _lib.call("eoship_memset", rt.handle, src.ptr, 1, C.c_size_t(nbytes))
    sink = DeviceBuffer(rt, blocks * 256 * 16)
    args = Args(src.ptr, sink.ptr, nbytes // 16)
    params = (C.c_void_p * 1)(C.cast(C.pointer(args), C.c_void_p))
    grid = (C.c_uint32 * 3)(blocks, 1, 1)
    block = (C.c_uint32 * 3)(256, 1, 1)
    try:
        for _ in range(2):
            _lib.call("eoship_launch", rt.handle, fn, grid, block, C.c_uint32(0), params)
        rt.sync()
        times = []
        for _ in range(reps):
            rt.mark(4)
            _lib.call("eoship_launch", rt.handle, fn, grid, block, C.c_uint32(0), params)
            rt.mark(5)
            times.append(rt.elapsed_ms(4, 5))
    finally:
        src.free()
        sink.free()
        _lib.call("eoship_module_unload", mod)
    ms = float(np.median(times))
    return {"bytes": nbytes, "ms": ms, "read_GBps": nbytes / (ms / 1e3) / 1e9}


def copy_calibration(rt, mb: int, reps: int = 5) -> dict:
    """Device-to-device copies of a known size: the reference kernel whose
    FETCH_SIZE / WRITE_SIZE counters scale the scan's in a --pmc run."""
    from eos_amd.runtime import DeviceBuffer
    from eos_amd import _lib
    import ctypes as C
    nbytes = mb * 1_000_000
    src = DeviceBuffer(rt, nbytes)
    dst = DeviceBuffer(rt, nbytes)
    rt.sync()
    rt.mark(4)
    for _ in range(reps):
        _lib.call("eoship_d2d", rt.handle, dst.ptr, src.ptr, C.c_size_t(nbytes))
    rt.mark(5)
    ms = rt.elapsed_ms(4, 5) / reps
    return {"bytes": nbytes, "ms": ms, "read_plus_write_GBps": 2 * nbytes / (ms / 1e3) / 1e9}



def mfma_ceiling(rt, iters: int = 400) -> dict:
    """Matrix-core rate and shader clock reached by a stream of independent
    MFMAs (eos_amd/csrc/kernels/probe_kernels.hip, 3 waves per SIMD, no VALU
    work) on three kinds of operand bytes: zeros, full-range random int8, and
    random f16 drawn N(0, 1). The clock falls under the power drawn by
    full-range operands, so the rate an int8 kernel can reach on real data
    is this ceiling, below the published dense peak (which assumes the top
    clock). Launch time from stream events; clock from s_memtime over
    s_memrealtime (100 MHz) inside each wave."""
    import ctypes as C
    from eos_amd import _lib
    from eos_amd.build import PROBE_PATH
    from eos_amd.runtime import DeviceBuffer

    if not os.path.exists(PROBE_PATH):
        raise RuntimeError(f"{PROBE_PATH} is missing: run python -m eos_amd.build")
    img = open(PROBE_PATH, "rb").read()
    mod = C.c_void_p()
    _lib.call("eoship_module_load", rt.handle, img, C.c_size_t(len(img)), C.byref(mod))
    cu = rt.info()["compute_units"]
    blocks = cu * 3
    waves = blocks * 4
    slots, frags = 64, 8
    words = slots * 2 * frags * 64 * 4
    rng = np.random.default_rng(0x5eed)
    operands = {
        "zeros": np.zeros(words, np.int32),
        "random_int8": rng.integers(-2**31, 2**31, words, dtype=np.int64).astype(np.int32),
        "random_f16": rng.standard_normal(words * 2).astype(np.float16).view(np.int32),
    }

    class Args(C.Structure):
        _fields_ = [("operands", C.c_void_p), ("sink", C.c_void_p), ("clocks", C.c_void_p),
                    ("iters", C.c_int)]

    sink = DeviceBuffer(rt, blocks * 256 * 4)
    clocks = DeviceBuffer(rt, waves * 16)
    grid = (C.c_uint32 * 3)(blocks, 1, 1)
    block = (C.c_uint32 * 3)(256, 1, 1)
    out = {"waves_per_simd": 3, "mfma_per_wave": iters * 64}
    try:
        for label, kname, kind, ops in (
                ("int8_zeros", "eos_probe_mfma_i8", "zeros", 2.0 * 32 ** 3),
                ("int8_random", "eos_probe_mfma_i8", "random_int8", 2.0 * 32 ** 3),
                ("f16_random", "eos_probe_mfma_f16", "random_f16", 2.0 * 32 * 32 * 16)):
            fn = C.c_void_p()
            _lib.call("eoship_function", mod, kname.encode(), C.byref(fn))
            src = DeviceBuffer.from_array(rt, operands[kind])
            args = Args(src.ptr, sink.ptr, clocks.ptr, iters)
            params = (C.c_void_p * 1)(C.cast(C.pointer(args), C.c_void_p))

            def launch():
                _lib.call("eoship_launch", rt.handle, fn, grid, block, C.c_uint32(0), params)

            for _ in range(3):
                launch()
            rt.sync()
            rt.mark(8)
            reps = 5
            for _ in range(reps):
                launch()
            rt.mark(9)
            ms = rt.elapsed_ms(8, 9) / reps
            clk = clocks.download(np.uint64, (waves, 2)).astype(np.float64)
            mhz = float(np.median(clk[:, 0] / (clk[:, 1] / 100.0)))
            total = waves * iters * 64 * ops
            out[label] = {"tops": total / (ms / 1e3) / 1e12, "clock_mhz": mhz, "ms": ms}
            src.free()
    finally:
        sink.free()
        clocks.free()
        _lib.call("eoship_module_unload", mod)
    return out


def tiny_leg(rt, reps: int, cpu: bool = True) -> dict:
    """Benchmark config c1 (examples/embed.eos): f16 token_embedding [30522, 256]
    and projection [256, 128], N(0, 0.02); 128 tokens; gather -> matmul ->
    row L2 normalize -> f16 [128, 128]. Latency-bound: one launch per call."""
    from eos_amd import datagen
    from eos_amd.encoder import TinyEmbed
    from eos_amd.runtime import DeviceBuffer

    V, D, E, T = 30522, 256, 128, 128
    table = (0.02 * datagen.normal(1, V * D)).astype(np.float16).reshape(V, D)
    proj = (0.02 * datagen.normal(101, D * E)).astype(np.float16).reshape(D, E)
    tokens = datagen.uniform_int(2, T, 0, V).astype(np.int32)
    m = TinyEmbed(rt, table, proj)
    d_tok = DeviceBuffer.from_array(rt, tokens)
    d_out = DeviceBuffer(rt, T * E * 2)
    for _ in range(20):
        m.embed_device(d_tok, T, d_out)
    rt.sync()
    rt.mark(8)
    for _ in range(reps):
        m.embed_device(d_tok, T, d_out)
    rt.mark(9)
    us = rt.elapsed_ms(8, 9) / reps * 1e3
    rt.profile_reset()
    rt.profile_select(None)
    rt.profile(True)
    for _ in range(reps):
        m.embed_device(d_tok, T, d_out)
    rt.sync()
    n_k, ms_k = rt.profile_read("eos_embed_tiny")
    rt.profile(False)
    kern_us = ms_k / max(n_k, 1) * 1e3
    # One call end to end from the host (tokens up, embeddings down).
    t0 = time.perf_counter()
    for _ in range(50):
        m.embed(tokens)
    host_us = (time.perf_counter() - t0) / 50 * 1e6
    touched = T * D * 2 + D * E * 2 + T * E * 2 + T * 4
    out = {
        "metric": "tiny embed calls/s (T = 128)",
        "value": 1e6 / us,
        "unit": "calls/s",
        "us_per_call": us,
        "tokens_per_s": T * 1e6 / us,
        "kernel_us": kern_us,
        "host_roundtrip_us_per_call": host_us,
        "config": {"workload": "tiny_embed_c1", "vocab": V, "dim": D, "out_dim": E, "tokens": T},
        "roofline": {"bound": "latency", "kernel": "eos_embed_tiny", "avg_launch_ms": kern_us / 1e3,
                     "bytes_per_launch": touched, "flops_per_launch": 2.0 * T * D * E,
                     "achieved_gbs": touched / (kern_us / 1e6) / 1e9 if kern_us > 0 else None},
    }
    if cpu:
        import oracle
        tf, pf = table.astype(np.float32), proj.astype(np.float32)
        n = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 2.0:
            oracle.tiny_embed(tf, pf, tokens)
            n += 1
        dt = (time.perf_counter() - t0) / n
        out["cpu_baseline"] = {
            "value": 1.0 / dt, "unit": "calls/s", "us_per_call": dt * 1e6,
            "tokens_per_s": T / dt, "cores": 1, "kind": "port",
            "sample": f"{n} calls in 2 s: single-threaded C restatement of gather + f32 "
                      "matmulTensor (k order) + normalizeRows",
            "cpu_model": _cpu_model()}
    for b in (d_tok, d_out):
        b.free()
    m.release()
    return out


def two_stage_leg(rt, steps: int, n: int) -> dict:
    """Two-stage retrieval on the c2 corpus shape as the promoted serving
    profile turboquant_ip_b4_overfetch200_fp16_rerank runs it
    (runtime/retrieval_turboquant.go:1500-1556): n x 384 unit Gaussian
    documents encoded on the device into the inner-product layout at bit
    width 4 (3-bit MSE codes + QJL sign bits + ResNorm + Norm, 200 B per
    vector), the top 200 by the inner-product estimate, then the f16 rerank
    of those 200 to the top 100 with the rank-100 rescue (gate fed bit width
    4). f16 rows: the same documents, converted on the device at bind."""
    from eos_amd import datagen
    from eos_amd.runtime import DeviceBuffer
    from eos_amd.turboquant import F16Sidecar, IPQuantizer, top_fp16_rerank_scores_device

    dim, bit_width, nq, k, over = 384, 4, 64, 100, 200
    mse_bits = bit_width - 1
    log("two-stage c2: generating documents, IP b4 encode, f16 rows")
    rng = np.random.default_rng(35)
    rot = np.linalg.qr(rng.standard_normal((dim, dim)))[0].astype(np.float32)
    sketch = rng.standard_normal((dim, dim)).astype(np.float32)
    cb, s_c = datagen.turboquant_codebook(mse_bits, dim)
    qz = IPQuantizer(rt, dim, mse_bits, cb, s_c, rot, sketch)
    row_bytes, sign_bytes = qz.row_bytes, qz.sign_bytes
    d_codes = DeviceBuffer(rt, n * row_bytes)
    d_signs = DeviceBuffer(rt, n * sign_bytes)
    d_rn = DeviceBuffer(rt, n * 4)
    d_nm = DeviceBuffer(rt, n * 4)
    side = F16Sidecar.allocate(rt, n, dim)
    import ctypes as C
    from eos_amd import _lib
    chunk = 131072
    for c0 in range(0, n, chunk):
        m = min(chunk, n - c0)
        x = rng.standard_normal((m, dim), dtype=np.float32)
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        dx = DeviceBuffer.from_array(rt, x)
        _lib.call("eoship_tq_ip_encode_device", rt.handle, C.byref(qz.spec), dx.ptr, C.c_int64(m),
                  d_codes.view(c0 * row_bytes, m * row_bytes).ptr,
                  d_signs.view(c0 * sign_bytes, m * sign_bytes).ptr,
                  d_rn.view(c0 * 4, m * 4).ptr, d_nm.view(c0 * 4, m * 4).ptr)
        side.fill_device(dx, c0, m)
        rt.sync()
        dx.free()
    idx = qz.bind(d_codes, d_signs, d_rn, d_nm)
    for b in (d_codes, d_signs, d_rn, d_nm):
        b.free()
    q = datagen.baseline_queries(nq, dim, 34)
    dq = DeviceBuffer.from_array(rt, q)
    dcid, dcs = DeviceBuffer(rt, nq * over * 8), DeviceBuffer(rt, nq * over * 4)
    dids, dsc = DeviceBuffer(rt, nq * k * 8), DeviceBuffer(rt, nq * k * 4)

    def step():
        idx.top_k_device(dq, nq, over, dcid, dcs)
        top_fp16_rerank_scores_device(side, dq, nq, dcid, dcs, over, k, bit_width, over, dids, dsc)

    for _ in range(3):
        step()
    rt.sync()
    rt.mark(6)
    for _ in range(steps):
        step()
    rt.mark(7)
    ms = rt.elapsed_ms(6, 7) / steps
    rt.profile_reset()
    rt.profile_select(None)
    rt.profile(True)
    for _ in range(10):
        step()
    rt.sync()
    kernels = {}
    for name in ("tq_ip_prepare", "tq_ipscan_sample", "tq_ip_threshold",
                 "tq_ipscan_filter", "tq_ip_rescore", "tq_ip_finalize", "tq_ipscan_dense",
                 "tq_ip_fallback_select",
                 "tq_fp16_rerank_dots", "tq_fp16_rerank_sort"):
        kernels[name] = rt.profile_read(name)[1] / 10
    filt = rt.profile_samples("tq_ipscan_filter")
    n_rr, ms_rr = rt.profile_read("tq_fp16_rerank")
    rt.profile(False)
    med = float(np.median(filt)) if len(filt) else 0.0
    bytes_per_launch = n * (row_bytes + sign_bytes + 8)
    # int8 ops of the high-half bound filter: per (query, vector, dimension)
    # a MAC in each of its two int8 passes (the MSE grid's and the QJL
    # grid's high halves); the exact scores it stands for take four (the low
    # halves too), reported beside it as the exact-equivalent rate.
    ops = 2.0 * 2 * nq * n * dim
    ops_exact = 2.0 * 4 * nq * n * dim
    avg = ms_rr / max(n_rr, 1)
    rr_bytes = nq * over * (dim * 2 + 12) + nq * dim * 4 + nq * k * 12
    out = {
        "metric": "two-stage retrieval queries/s (IP b4 top-200 + f16 rerank top-100)",
        "value": nq / (ms / 1e3),
        "unit": "queries/s",
        "ms_per_batch": ms,
        "vectors_scored_per_s": n * nq / (ms / 1e3),
        "config": {"workload": "turboquant_two_stage_c2", "n": n, "dim": dim,
                   "bit_width": bit_width, "mse_bits": mse_bits, "queries": nq,
                   "overfetch": over, "k": k,
                   "profile": "turboquant_ip_b4_overfetch200_fp16_rerank",
                   "bytes_per_vector": row_bytes + sign_bytes + 8},
        "breakdown_ms": kernels,
        "roofline": {"kernel": "tq_ipscan_filter", "median_launch_ms": med,
                     "bytes_per_launch": bytes_per_launch,
                     "hbm_gbs": bytes_per_launch / (med / 1e3) / 1e9 if med > 0 else None,
                     "hbm_frac": bytes_per_launch / (med / 1e3) / 1e9 / HBM_PEAK_GBS if med > 0 else None,
                     "int8_ops_per_launch": ops,
                     "achieved": ops / (med / 1e3) / 1e12 if med > 0 else None,
                     "peak": INT8_PEAK_TOPS, "unit": "TOP/s (int8)",
                     "frac": ops / (med / 1e3) / 1e12 / INT8_PEAK_TOPS if med > 0 else None,
                     "exact_int8_ops_per_launch": ops_exact,
                     "exact_equivalent_tops": ops_exact / (med / 1e3) / 1e12 if med > 0 else None,
                     "exact_equivalent_frac": (ops_exact / (med / 1e3) / 1e12 / INT8_PEAK_TOPS
                                               if med > 0 else None),
                     "bound": "mfma"},
        "rerank": {"kernel": "tq_fp16_rerank", "bound": "latency", "avg_launch_ms": avg,
                   "launches": n_rr, "bytes_per_launch": rr_bytes,
                   "achieved_gbs": rr_bytes / (avg / 1e3) / 1e9 if avg > 0 else None},
    }
    for b in (dq, dcid, dcs, dids, dsc):
        b.free()
    side.buf.free()
    idx.release()
    qz.release()
    return out

def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--queries", type=int, default=64)
    ap.add_argument("--k", type=int, default=100)
    ap.add_argument("--streams", type=int, default=3, choices=(1, 2, 3, 4),
                    help="query batches in flight (one stream each) in the timed region; "
                         "three measured best (1: 0.100, 2: 0.085, 3: 0.078, 4: 0.089 ms per step)")
    ap.add_argument("--cpu-sample-queries", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-encoder", action="store_true")
    ap.add_argument("--skip-tq", action="store_true", help="profiling runs of the encoder only")
    ap.add_argument("--skip-maxsim", action="store_true")
    ap.add_argument("--skip-two-stage", action="store_true")
    ap.add_argument("--maxsim-steps", type=int, default=5)
    ap.add_argument("--encoder-steps", type=int, default=5)
    ap.add_argument("--encoder-configs", default="c3,c4", help="comma list of c3, c4")
    ap.add_argument("--copy-calibration-mb", type=int, default=1024)
    ap.add_argument("--skip-tiny", action="store_true")
    ap.add_argument("--shard-n", type=int, default=125_000,
                    help="c2 at one GPU's shard of an 8-GPU job (0: skip)")
    ap.add_argument("--tiny-reps", type=int, default=2000)
    ap.add_argument("--skip-mfma-ceiling", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the scan would shard by corpus rows, each GPU scoring its own rows, with one top-k merge)",
              file=sys.stderr)
        return 2

    from eos_amd.runtime import Runtime

    rt = Runtime(0)
    info = rt.info()
    log(f"device {info}")
    out = {
        "metric": METRIC,
        "unit": "vectors scored/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes x int16 query (int8 MFMA, exact i32), f32 scores",
        "data": "synthetic (seeded splitmix64: uniform 4-bit codes, lognormal(0,0.25) norms, "
                "QR rotation, unit Gaussian queries)",
    }
    if not args.skip_tq:
        out.update(tq_leg(rt, args))
        if args.copy_calibration_mb > 0:
            # Achievable HBM: a device-to-device copy of a known size beside
            # the vendor peak.
            cal = copy_calibration(rt, args.copy_calibration_mb)
            out["copy_calibration"] = cal
            # The scan only reads: its measured peak is a read-only stream,
            # over a buffer past the 256 MB Infinity Cache (HBM) and over
            # the corpus's own size (which the cache can partly hold).
            rd = read_calibration(rt, args.copy_calibration_mb)
            rd_corpus = read_calibration(rt, out["roofline"]["bytes_per_launch"] // 1_000_000)
            out["read_calibration"] = {"hbm": rd, "corpus_size": rd_corpus}
            roof = out["roofline"]
            roof["peak_measured_read_only"] = rd["read_GBps"]
            roof["frac_measured_read_only"] = roof["achieved"] / rd["read_GBps"]
            roof["peak_measured_read_only_corpus_size"] = rd_corpus["read_GBps"]
            roof["peak_measured_copy"] = cal["read_plus_write_GBps"]
            roof["frac_measured_copy"] = roof["achieved"] / cal["read_plus_write_GBps"]
    if not args.skip_tq and args.shard_n > 0:
        log(f"c2 shard ({args.shard_n} vectors)")
        out["tq_shard8_c2"] = tq_shard_leg(rt, args.shard_n, args.queries, args.k, args.steps,
                                           args.warmup)
    ceiling = None
    if not args.skip_mfma_ceiling and not (args.skip_encoder and args.skip_maxsim):
        log("MFMA ceiling probe")
        ceiling = mfma_ceiling(rt)
        out["mfma_ceiling"] = ceiling
    if not args.skip_tiny:
        log("tiny c1")
        out["tiny_c1"] = tiny_leg(rt, args.tiny_reps, cpu=not args.no_cpu_baseline)
    if not args.skip_encoder:
        for name in args.encoder_configs.split(","):
            log(f"encoder {name}")
            out[f"encoder_{name}"] = encoder_leg(rt, args.encoder_steps, name,
                                                 cpu=not args.no_cpu_baseline)
            if ceiling is not None:
                # The forward's flops split over int8 MFMAs (QKV, FFN-up) and
                # f16 MFMAs (O, FFN-down, attention): the time each share
                # would take at its clock-limited ceiling.
                roof = out[f"encoder_{name}"]["roofline"]
                sh = roof["int8_share_of_flops"]
                ceil = 1.0 / (sh / ceiling["int8_random"]["tops"]
                              + (1.0 - sh) / ceiling["f16_random"]["tops"])
                roof["ceiling_mixed_random"] = ceil
                roof["frac_of_ceiling"] = roof["achieved"] / ceil
    if not args.skip_maxsim:
        out["maxsim_c5"] = maxsim_leg(rt, args.maxsim_steps, cpu=not args.no_cpu_baseline)
        if ceiling is not None:
            # Against the rate full-range int8 operands allow (clock-limited).
            roof = out["maxsim_c5"]["roofline"]
            roof["ceiling_int8_random"] = ceiling["int8_random"]["tops"]
            roof["frac_of_ceiling"] = roof["achieved"] / ceiling["int8_random"]["tops"]
    if not args.skip_two_stage:
        log("two-stage c2")
        out["two_stage_c2"] = two_stage_leg(rt, args.maxsim_steps * 4, args.n)
    out["device"] = info
    rt.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
