"""compress-zip on one MI355X: compress tokens/s at L4 (512-token chunks).

One step = the whole workload compressed on the device: every chunk goes
through the batched causal prefill (int8 MFMA GEMMs, exact attention), the
fused logits -> CDF stage and the arithmetic coder, with the tokens already
resident in HBM.  Prints one JSON line (see the repository's bench contract).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "compress-zip_amd"))

import numpy as np  # noqa: E402

# MI355X published peaks (dense)
PEAK_INT8_TOPS = 5000.0     # TOP/s
PEAK_HBM_GBS = 8000.0       # GB/s

# The commits the two profile-derived constants below were measured at (they go
# stale when the kernels change; the bench line carries these names with them).
TRAFFIC_PROFILED_AT = "da916f6"
VALU_PROFILED_AT = "da916f6"
# HBM bytes per token (read + write) of each kernel on the text workload, from
# two rocprofv3 --pmc runs (FETCH_SIZE x2.0, WRITE_SIZE x1.0: the factors a
# plain 256 MiB copy calibrates); profiles/traffic_v001_ctx512_text.md
TRAFFIC_B_PER_TOKEN = {"attention": 513 + 384, "qkv_table": 12 + 512, "gemm_o_norm": 396 + 1152,
                       "ffn": 1408 + 386, "gemm_down_norm": 1946 + 384, "gemm_up": 677 + 1024, "head_cdf": 389 + 8}
TRAFFIC_WORKLOADS = ("v001_L4_ctx512_text64MiB",)
# Prefill attention: wave64 VALU instructions (MFMA excluded) per 16-row tile (64 keys, or
# 32 for a row block's last tile when its visible keys end in the first half), from
# SQ_INSTS_VALU - SQ_INSTS_VALU_MFMA_I8 on the same workload
# (profiles/counters_compress_v001_ctx512_text8Mtok.md); the VALU issue peak is one wave64
# instruction per 4 cycles per SIMD: 1024 SIMDs x 2.4 GHz / 4.
ATTN_VALU_PER_TILE = {"v001_L4_ctx512_text64MiB": 960}
PEAK_VALU_GINST = 1024 * 2.4 / 4 * 1e9 / 1e9

WORKLOADS = {
    # shipped model, level 4 (512-token chunks), 64 MiB of seeded synthetic text
    "v001_L4_ctx512_text64MiB": dict(model="shipped", chunk=512, text_bytes=64 << 20),
    # shipped model, level 4, Zipf(1.1) token ids (no tokenizer step)
    "v001_L4_ctx512_zipf16M": dict(model="shipped", chunk=512, ids=16 << 20),
    # random-init d512 / 8 layers / 8 heads, 2 KV heads / F 2048 / V 1024, level 5
    # (1024-token chunks), 16M Zipf ids, in the reference's KV semantics and in GQA
    "d512L8_L5_ctx1024_zipf16M": dict(model="d512_l8", chunk=1024, ids=16 << 20, kv="rust_compat"),
    "d512L8_L5_ctx1024_zipf16M_gqa": dict(model="d512_l8", chunk=1024, ids=16 << 20, kv="gqa"),
    # the same model decoding 4096 concurrent streams of 512 tokens (its compress
    # leg codes them at level 4)
    "d512L8_decode_4096x512": dict(model="d512_l8", chunk=512, ids=4096 * 512, kv="rust_compat"),
    # random-init d768 / 12 layers / 12 heads, 4 KV heads / F 3072 / V 8192, one
    # 4096-token context per chunk, 8M Zipf ids; GQA only (attention.rs:172 rejects 12 heads)
    "d768L12_ctx4096_zipf8M_gqa": dict(model="d768_l12", chunk=4096, ids=8 << 20, kv="gqa"),
}
DEFAULT = "v001_L4_ctx512_text64MiB"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_tokens(wl, weights, vocab):
    """Token ids of the workload and, for text workloads, the text and tokenizer."""
    import czip_amd
    from czip_amd import synth
    if "ids" in wl:
        return synth.zipf_ids(wl["ids"], vocab, seed=7), None, None
    t = time.perf_counter()
    text = synth.synthetic_text(wl["text_bytes"], seed=1234)
    tk = czip_amd.Tokenizer(weights)
    t1 = time.perf_counter()
    ids = tk.encode(text, threads=min(16, len(os.sched_getaffinity(0))))
    log(f"text {len(text)} B generated in {t1 - t:.1f} s, tokenized in {time.perf_counter() - t1:.1f} s")
    return ids, text, tk


def gemm_ops_per_token(cfg, kv_mode):
    d, F, V, G = cfg["d_model"], cfg["d_ff"], cfg["vocab_size"], cfg["n_kv_heads"]
    qkv_n = d + 2 * G * 64 if kv_mode == 1 else d + 128
    per_layer = {"gemm_qkv": qkv_n * d, "gemm_o": d * d, "gemm_o_norm": d * d, "gemm_up": 2 * F * d,
                 "gemm_down": d * F, "gemm_down_norm": d * F, "ffn": 2 * F * d + d * F}
    out = {k: 2 * v * cfg["n_layers"] for k, v in per_layer.items()}
    # layer 0's QKV projection is a per-token table (qkv_table: RoPE and scatter only)
    out["gemm_qkv"] = 2 * qkv_n * d * (cfg["n_layers"] - 1)
    out["gemm_head"] = 2 * V * d
    out["head_cdf"] = 2 * V * d
    return out


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model_path, tokens, chunk, budget_s=15.0, kv_mode=0, extra_chunks=()):
    """Oracle (C restatement of the Rust chunk loop) on the host cores.
    Returns (baseline record, {chunk index: oracle bytes}) for the timed
    sample (the first chunks) plus `extra_chunks`, coded after the timing."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    try:
        lib_path = oracle.build(native=True)
        kind_note = "gcc -O3 -march=native"
    except Exception:
        lib_path = oracle.LIB_PATH
        kind_note = "gcc -O3 -march=x86-64-v3"
    L = oracle.load(lib_path)
    m = oracle.Model.from_file(model_path, kv_mode, lib_handle=L)
    cores = min(16, len(os.sched_getaffinity(0)))
    nchunks = len(tokens) // chunk
    # calibrate with one chunk per thread, then size the sample to the budget
    k0 = min(nchunks, cores)
    t = time.perf_counter()
    m.compress_many(tokens[:k0 * chunk], chunk, threads=cores)
    dt0 = time.perf_counter() - t
    per_round = max(dt0, 1e-3)
    rounds = max(1, int(budget_s / per_round))
    k = min(nchunks, cores * rounds)
    t = time.perf_counter()
    first = m.compress_many(tokens[:k * chunk], chunk, threads=cores)
    dt = time.perf_counter() - t
    coded = dict(enumerate(first))
    extra = [c for c in extra_chunks if c not in coded]
    log(f"cpu baseline: {k} chunks in {dt:.1f} s; coding {len(extra)} more for the parity sample")
    if extra:
        sample = np.concatenate([tokens[c * chunk:(c + 1) * chunk] for c in extra])
        # every extra chunk but the job's last is full, so chunk boundaries line up
        for c, b in zip(extra, m.compress_many(sample, chunk, threads=cores)):
            coded[c] = b
    rec = {"value": round(k * chunk / dt, 1), "unit": "tok/s", "cores": cores, "kind": "port",
           "cpu_model": cpu_model(), "nproc": os.cpu_count(),
           "sample": f"first {k} chunks x {chunk} tokens ({k * chunk} tokens) of the same workload, "
                     f"{cores} threads, C oracle ({kind_note}), {dt:.1f} s"}
    return rec, coded


def ceilings():
    """The measured ceilings beside the published peaks: a streaming copy of
    1 GiB (read + write bytes over time) and dense int8 MFMA chains with no
    memory traffic (8 waves per SIMD) of both int8 shapes, from
    libczip_ceiling.so.  int8_mfma_tops is the faster shape's (32x32x32);
    the path's kernels issue 16x16x64, whose own ceiling is reported beside it."""
    import ctypes as C
    from czip_amd import build as b
    L = C.CDLL(b.CEILING_LIB_PATH)
    L.czc_copy_gbs.argtypes = [C.c_size_t, C.c_int, C.POINTER(C.c_double)]
    L.czc_read_gbs.argtypes = [C.c_size_t, C.c_int, C.POINTER(C.c_double)]
    L.czc_mfma_i8_tops.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]
    best = {"copy": 0.0, "read": 0.0, 32: 0.0, 16: 0.0}
    v = C.c_double()
    for _ in range(3):  # the best of three: the clock under a long MFMA loop varies between runs and boxes
        if L.czc_copy_gbs(1 << 30, 10, C.byref(v)):
            raise SystemExit("copy ceiling probe failed")
        best["copy"] = max(best["copy"], v.value)
        if L.czc_read_gbs(1 << 30, 10, C.byref(v)):
            raise SystemExit("read ceiling probe failed")
        best["read"] = max(best["read"], v.value)
        for shape, iters in ((32, 4000), (16, 2000)):
            if L.czc_mfma_i8_tops(shape, iters, 8, C.byref(v)):
                raise SystemExit("MFMA ceiling probe failed")
            best[shape] = max(best[shape], v.value)
    return {"hbm_copy_gbs": round(best["copy"], 1), "hbm_read_gbs": round(best["read"], 1),
            "int8_mfma_tops": round(best[32], 1),
            "int8_mfma_16x16x64_tops": round(best[16], 1),
            "copy": "1 GiB device-to-device copy kernel, 16-byte loads/stores, 4 workgroups per CU, 10 timed passes, "
                    "best of 3; read: 1 GiB summed with 16-byte loads, 8 workgroups per CU",
            "mfma": "v_mfma_i32_32x32x32_i8, 4 independent chains per wave (16x16x64: 16 chains), "
                    "8 waves per SIMD, no memory traffic, best of 3"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decompress", action="store_true", help="skip the decompress leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--tokens", type=int, default=0, help="truncate the workload (profiling runs only)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); chunks would shard across GPUs "
              f"by chunk range with no communication during the compute", file=sys.stderr)
        sys.exit(2)
    import czip_amd
    if not os.path.exists(czip_amd.LIB_PATH):
        from czip_amd import build as b
        b.build()
    wl = WORKLOADS[args.workload]
    if wl["model"] == "shipped":
        model_path = os.path.join(ROOT, "models", "v001_eng.czm")
        model_name = "v001_eng.czm"
    else:
        # random-init weights of the named shape (seeded), written once per run
        import tempfile
        from czip_amd import synth
        model_path = os.path.join(tempfile.mkdtemp(prefix="czip_bench_"), wl["model"] + ".czm")
        synth.write_random_model(model_path, seed=2024, **synth.MODEL_SHAPES[wl["model"]])
        model_name = f"random-init {wl['model']} (seed 2024)"
    kv_name = wl.get("kv", "rust_compat")
    kv_mode = czip_amd.KV_GQA if kv_name == "gqa" else czip_amd.KV_RUST_COMPAT
    weights = czip_amd.ModelWeights(model_path, kv_mode)
    cfg = weights.config
    tokens, text, tokenizer = make_tokens(wl, weights, cfg["vocab_size"])
    if args.tokens and args.tokens < tokens.size:
        tokens = tokens[:args.tokens]
        text = None  # a token prefix: the round trip is checked on the ids only
    chunk = wl["chunk"]
    n = int(tokens.size)
    log(f"workload {args.workload}: {n} tokens, chunk {chunk}")
    model = czip_amd.Model(weights, device=0)
    ceil = ceilings()
    log(f"ceilings: copy {ceil['hbm_copy_gbs']:.0f} GB/s, int8 MFMA {ceil['int8_mfma_tops']:.0f} TOP/s")
    t_plan = time.perf_counter()
    job = model.compress_plan(tokens, chunk)  # device buffers + host-to-device copy of the tokens
    plan_ms = (time.perf_counter() - t_plan) * 1000.0
    for _ in range(args.warmup):
        job.run()
    # the rate: K steps with no per-kernel instrumentation
    t0 = time.perf_counter()
    for _ in range(args.steps):
        job.run()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1000.0 / args.steps
    value = n / (ms / 1000.0)
    log(f"compress: {ms:.1f} ms per step, {value / 1e6:.2f} M tok/s")
    # the per-kernel breakdown: one more step with HIP events around every launch
    model.reset_stats()
    model.set_profiling(True)
    job.run()
    model.set_profiling(False)
    t_fetch = time.perf_counter()
    data, offs = job.fetch_packed()
    fetch_ms = (time.perf_counter() - t_fetch) * 1000.0
    job.free()
    raw = data.tobytes()
    chunks = [raw[offs[c]:offs[c + 1]] for c in range(len(offs) - 1)]
    coded = int(offs[-1])
    e2e = {"value": round(n / ((plan_ms + ms + fetch_ms) / 1000.0), 1), "unit": "tok/s",
           "plan_ms": round(plan_ms, 2), "run_ms": round(ms, 2), "fetch_ms": round(fetch_ms, 2),
           "span": "device buffers + token upload, one step, coded bytes back to the host (packed)"}
    prof_steps = 1

    # per-kernel breakdown from HIP events on the context stream
    ops = gemm_ops_per_token(cfg, kv_mode)
    nrows = ((n + chunk - 1) // chunk) * chunk
    kernels = {}
    for name in ["prep", "embed_norm", "qkv_table", "gemm_qkv", "attention", "gemm_o", "gemm_o_norm", "row_norm", "gemm_up",
                 "gemm_down", "gemm_down_norm", "ffn", "gemm_head", "cdf", "head_cdf", "encode"]:
        launches, tot = model.kernel_stats(name)
        if launches:
            kernels[name] = {"launches": launches, "avg_ms": tot / launches, "ms_per_step": tot / prof_steps}
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    gemm_ms = sum(kernels[k]["ms_per_step"] for k in kernels if k in ops)
    gemm_tops = sum(ops[k] for k in kernels if k in ops) * nrows / (gemm_ms / 1000.0) / 1e12 if gemm_ms else 0.0
    if dom.startswith("gemm"):
        per_launch = ops[dom] * nrows / (kernels[dom]["launches"] / prof_steps)
        ach = per_launch / (kernels[dom]["avg_ms"] / 1000.0) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_INT8_TOPS, 4), "traffic": None, "kernel": dom}
    elif dom == "attention":
        H, T = cfg["n_heads"], chunk
        flops_per_chunk = sum(2 * 2 * H * 64 * (p + 1) for p in range(T)) * cfg["n_layers"]
        per_launch = flops_per_chunk * (nrows // T) / (kernels[dom]["launches"] / prof_steps)
        ach = per_launch / (kernels[dom]["avg_ms"] / 1000.0) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 3), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_INT8_TOPS, 5), "traffic": None, "kernel": dom}
        if args.workload in ATTN_VALU_PER_TILE and not args.tokens:
            # the bound it actually hits: VALU issue (16-row x 64-key tiles, causal)
            nq16 = (T + 15) // 16
            tiles_chunk = H * sum((16 * b + 15) // 64 + 1 for b in range(nq16))
            tiles_launch = tiles_chunk * (nrows // T) / (kernels[dom]["launches"] / prof_steps)
            gi = ATTN_VALU_PER_TILE[args.workload] * tiles_launch / (kernels[dom]["avg_ms"] / 1000.0) / 1e9
            roof["valu"] = {"per_tile": ATTN_VALU_PER_TILE[args.workload], "tiles_per_launch": round(tiles_launch),
                            "achieved": round(gi, 1), "peak": PEAK_VALU_GINST, "unit": "G wave64 VALU inst/s",
                            "frac": round(gi / PEAK_VALU_GINST, 4)}
    else:
        V = cfg["vocab_size"]
        per_launch = (4 * V + 8) * nrows / (kernels[dom]["launches"] / prof_steps)
        ach = per_launch / (kernels[dom]["avg_ms"] / 1000.0) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None, "kernel": dom}

    if args.workload in TRAFFIC_WORKLOADS and roof["kernel"] in TRAFFIC_B_PER_TOKEN:
        per_launch_tokens = n / (kernels[dom]["launches"] / prof_steps)
        roof["traffic"] = round(TRAFFIC_B_PER_TOKEN[roof["kernel"]] * per_launch_tokens)
        roof["traffic_source"] = (f"rocprofv3 FETCH_SIZE/WRITE_SIZE per token (profiled at {TRAFFIC_PROFILED_AT}) "
                                  f"x tokens per launch")
    if "valu" in roof:
        roof["valu"]["profiled_at"] = VALU_PROFILED_AT
    # the same rate against the measured ceiling of its resource
    roof["frac_of_measured"] = round(roof["achieved"] / (ceil["int8_mfma_tops"] if roof["bound"] == "mfma"
                                                         else ceil["hbm_copy_gbs"]), 5)

    # decompress leg: the chunks just coded, decoded back on the device as
    # concurrent streams (one token per stream per step), checked for identity
    dec = None
    if not args.no_decompress:
        ntoks = [min(chunk, n - c * chunk) for c in range(len(chunks))]
        djob = model.decompress_plan(chunks, ntoks)
        log(f"decompress: {len(chunks)} streams ...")
        # the rate comes from a run without events (a decode job launches
        # ~7 kernels per step); the per-kernel times from a second run of the
        # same job with HIP events around every launch
        t0 = time.perf_counter()
        djob.run()
        t1 = time.perf_counter()
        back = djob.fetch()
        if not np.array_equal(back, tokens):
            raise SystemExit("decompressed tokens differ from the input")
        if text is not None and tokenizer.decode_bytes(back) != text:
            raise SystemExit("detokenized output differs from the input text")
        log(f"decompress: {(t1 - t0):.2f} s, {n / (t1 - t0) / 1e6:.3f} M tok/s, tokens identical; per-kernel run ...")
        model.reset_stats()
        model.set_profiling(True)
        djob.run()
        model.set_profiling(False)
        if not np.array_equal(djob.fetch(), tokens):
            raise SystemExit("decompressed tokens differ from the input (profiled run)")
        djob.free()
        dk = {}
        for name in ["dec_init", "dec_prep", "embed_norm", "qkv_table", "gemm_qkv", "attn_decode", "gemm_o", "gemm_o_norm",
                     "row_norm", "gemm_up", "gemm_down", "gemm_down_norm", "ffn", "head_dec", "gemm_head", "cdf_decode"]:
            launches, tot = model.kernel_stats(name)
            if launches:
                dk[name] = {"ms": round(tot, 3), "launches": launches}
        dec = {"value": round(n / (t1 - t0), 1), "unit": "tok/s", "ms": round((t1 - t0) * 1000, 2),
               "streams": len(chunks), "roundtrip_exact": True, "kernels": dk}
        if "attn_decode" in dk:
            # decode attention is HBM-bound: per stream-step, the cached K and V
            # of every key so far (128 B per key and KV head) + q in + out
            KH = cfg["n_kv_heads"] if kv_mode == czip_amd.KV_GQA else 1
            D = cfg["n_heads"] * 64
            keys = sum(t * (t + 1) // 2 for t in ntoks)
            alg = cfg["n_layers"] * (keys * KH * 128 + n * 2 * D)
            gbs = alg / (dk["attn_decode"]["ms"] / 1000.0) / 1e9
            dec["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                               "frac": round(gbs / PEAK_HBM_GBS, 4), "kernel": "attn_decode",
                               "algorithmic_bytes": alg, "frac_of_measured": round(gbs / ceil["hbm_read_gbs"], 4),
                               "measured_peak": "hbm_read_gbs"}

    cpu = None
    parity = None
    if not args.no_cpu:
        log("cpu baseline ...")
        nch = len(chunks)
        # a strided sample over the whole job, the last (ragged) chunk and the
        # last sub-batch included, checked against the oracle besides the timed prefix
        extra = sorted(set(np.linspace(0, nch - 1, 24).astype(int).tolist()) | {nch - 1})
        cpu, ref = cpu_baseline(model_path, tokens, chunk, args.cpu_budget, kv_mode, extra)
        bad = [c for c, b in ref.items() if chunks[c] != b]
        parity = {"chunks": len(ref), "mismatches": len(bad), "first_mismatch": bad[0] if bad else None,
                  "against": "oracle bytes of the timed CPU sample + 24 chunks strided over the job"}
    line = {
        "metric": ("compress tok/s (bit-exact .czip payload) at L4 ctx512, 1 GPU" if args.workload == DEFAULT
                   else f"compress tok/s (bit-exact .czip payload), {args.workload}, 1 GPU"),
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": args.workload, "model": model_name, "chunk_tokens": chunk, "tokens": n,
                   "text_bytes": len(text) if text is not None else None,
                   "chunks": len(chunks), "kv_mode": kv_name, "parallelism": "chunks"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "parity_sample": parity,
        "e2e": e2e,
        "decompress": dec,
        "gemm_int8_tops": round(gemm_tops, 2),
        "gemm_int8_frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
        "gemm_int8_frac_of_measured": round(gemm_tops / ceil["int8_mfma_tops"], 4),
        "ceilings": ceil,
        "coded_bytes": coded,
        "kernels": {k: {"avg_ms": round(v["avg_ms"], 4), "ms_per_step": round(v["ms_per_step"], 3),
                        "launches_per_step": v["launches"] // prof_steps} for k, v in kernels.items()},
    }
    if cpu:
        line["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    print(json.dumps(line), flush=True)
    if parity and parity["mismatches"]:
        log(f"parity sample: {parity['mismatches']} of {parity['chunks']} chunks differ from the oracle")
        sys.exit(1)


if __name__ == "__main__":
    main()
