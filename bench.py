"""Headline benchmark: encoder tokens/s of indecis's int8 ModernBERT-base
forward pass ("cfg4") on one MI355X, plus the
fraction of the int8 MFMA peak its kernels reach.

A step is one EncodeSeqs pass over the whole batch: 256 sequences with
lengths uniform in [64, 512] (seeded), ids uniform over the 50,368-token
vocabulary, packed end to end by cumulative offsets, random-init int8
weights of the ModernBERT-base shape (H 768, 22 layers, 12 heads, GeGLU
2x1152). The ids are already in HBM when the timed region starts and the
pooled [256, 768] output stays there (ixh_encode_device).

A large batch runs as token-balanced parts on several streams (the
library's default: two from 4,096 tokens on), so kernels of the parts
overlap; `value` and `ms_per_step` are measured that way. `roofline` is for the kernel class with
the most GPU time in one untimed pass of the batch as one part; it is
measured over K further timed steps with the batch as one part (the kernel
running alone), with that class's launches (only) bracketed by timing-only
HIP events on the library's stream: `achieved` is its algorithmic int8 ops
(or HBM bytes) per launch over their average duration.
`roofline_concurrent` is the same class inside the headline timed region.
`traffic` comes from a committed rocprofv3 PMC summary of that kernel
(profiles/pmc_<kernel>.json) when one matches, else null. `kernels` is the
per-class breakdown of the untimed pass.
`cpu_baseline` times the C restatement of the reference (oracle/, test
infrastructure) on a bounded sample of the same batch on the host cores.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_INT8_OPS = 5.0e15   # MI355X dense int8 MFMA, ops/s
PEAK_HBM = 8.0e12        # MI355X HBM3E, bytes/s

WORKLOADS = {
    # name: (model, batch, min length, max length)
    "cfg4": ("base", 256, 64, 512),
    "cfg3": ("small", 256, 16, 256),
    "cfg5": ("base", 8, 8192, 8192),
    # not a BASELINE config: cfg4's batch at the reference's own backbone
    # width (bekko a8m: hidden 384, 6 heads, MLP 2 x 1152; 22 layers as cfg4)
    "w384": ("bekko", 256, 64, 512),
}


def make_inputs(np, vocab, B, lo, hi, seed=20261201):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=B)
    seqs = [rng.integers(0, vocab, size=int(n), dtype=np.int32) for n in lens]
    return seqs


def _host_info():
    """The host CPU model and the Go toolchain, if any (the reference itself
    needs Go 1.27 with GOEXPERIMENT=simd)."""
    import shutil
    import subprocess
    cpu = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    go = shutil.which("go")
    ver = None
    if go:
        try:
            ver = subprocess.run([go, "version"], capture_output=True, text=True, timeout=20).stdout.strip()
        except (OSError, subprocess.SubprocessError):
            ver = "go present, version unreadable"
    return {"cpu": cpu, "go": ver}


def cpu_baseline(np, weights, seqs, max_tokens):
    """Times the CPU restatement of the reference's int8 path (oracle/:
    OpenMP, MatMul8N and Attn8's products on VPDPBUSD tiles as the
    reference's VNNI kernels compute them, bit-identical to the checker)
    on the first sequences of the batch up to max_tokens tokens, on every
    host thread, then on one thread over a sixth of that sample."""
    from oracle import oracle as orc

    def sample_of(limit):
        sample, n = [], 0
        for s in seqs:
            if n + len(s) > limit and sample:
                break
            sample.append(s)
            n += len(s)
        return sample, n

    om = orc.OracleModel(weights, lanes=8)
    level = orc.set_gemm(1)
    L = orc.lib()
    cores = L.ixo_max_threads()
    res = {}
    try:
        for threads, limit in ((cores, max_tokens), (1, max(512, max_tokens // 6))):
            L.ixo_set_threads(threads)
            sample, n = sample_of(limit)
            om.encode_seqs(sample[:1])  # warm-up
            t0 = time.perf_counter()
            om.encode_seqs(sample)
            dt = time.perf_counter() - t0
            res[threads] = (n, len(sample), dt)
    finally:
        L.ixo_set_threads(cores)
        orc.set_gemm(0)
    n, b, dt = res[cores]
    n1, b1, dt1 = res[1]
    kind = {2: "AVX-512 VNNI", 1: "AVX-VNNI", 0: "no VNNI: plain loops"}[level]
    return {"value": round(n / dt, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"first {b} sequences ({n} tokens) of the same batch, {dt:.1f} s; C restatement of "
                      f"linalg/modernbert int8 with {kind} 6x16 tiles (OpenMP), not the Go reference",
            "single_core": {"value": round(n1 / dt1, 2), "unit": "tokens/s",
                            "sample": f"first {b1} sequences ({n1} tokens), {dt1:.1f} s"},
            "host": _host_info()}


def load_traffic(kernel, workload):
    path = os.path.join(ROOT, "profiles", f"pmc_{kernel}.json")
    if not os.path.exists(path):
        return None
    try:
        d = json.load(open(path))
    except (OSError, ValueError):
        return None
    if d.get("workload") != workload or d.get("kernel_class") != kernel:
        return None
    return d.get("hbm_bytes_per_launch")


def serving(np, model, cfg, args):
    """WithBatching under load (model.go:136-160): `clients` threads each
    send `requests` requests of one sequence (U[16,128] tokens, host ids in,
    pooled row out), first as direct concurrent EncodeSeqs calls, then
    through the batcher; one JSON line with both rates."""
    import threading
    from indecis_amd.modernbert import Batcher
    rng = np.random.default_rng(7)
    reqs = [[rng.integers(0, cfg.vocab, size=int(rng.integers(16, 129)), dtype=np.int32)]
            for _ in range(args.clients * args.requests)]
    tokens = sum(len(r[0]) for r in reqs)

    def run(fn):
        def burst(step):
            def client(k):
                for i in range(k, len(reqs), step):
                    fn(reqs[i])
            ts = [threading.Thread(target=client, args=(k,)) for k in range(args.clients)]
            t0 = time.perf_counter()
            for t in ts:
                t.start()
            for t in ts:
                t.join()
            return time.perf_counter() - t0
        burst(len(reqs))  # warm-up: one request per client, concurrently (workspaces)
        return burst(args.clients)

    direct = run(model.encode_seqs)
    bat = Batcher(model)
    batched = run(bat.encode_seqs)
    passes, served = bat.stats()
    bat.close()
    n = len(reqs)
    print(json.dumps({
        "metric": "serving: single-sequence requests/s from concurrent clients",
        "unit": "requests/s", "higher_is_better": True, "n_gpus": 1, "data": "synthetic",
        "config": {"workload": f"ModernBERT-{'base' if cfg.hidden == 768 else 'small'}-shaped int8 encoder, "
                               f"{args.clients} client threads x {args.requests} requests of 1 sequence "
                               f"(U[16,128] tokens), pooled output to the host",
                   "requests": n, "tokens": tokens},
        "direct": {"value": round(n / direct, 1), "tokens_per_s": round(tokens / direct, 1)},
        "batcher": {"value": round(n / batched, 1), "tokens_per_s": round(tokens / batched, 1),
                    "requests_per_pass": round(served / max(passes, 1), 2),
                    "note": "library defaults: 2 workers, 65536 tokens per pass"},
    }), flush=True)


def spans(np, model, cfg, seqs, args):
    """The token-level spans head of cfg3 and cfg5 (BIO over 4 span types:
    9 logits a token, spanTagCount spans.go:125; logits spans.go:449-459)
    on every token of the batch, in the encoder pass (ixh_encode_heads:
    host ids in, host float64 logits out, mean pooling as infer pools with
    Spans questions, spans.go:466-476). Reports the call's rate (the
    library's default split) and the head kernel's HBM rate from its HIP
    events with the batch as one part (its algorithmic bytes: each token's
    float32 state in, 9 float64 logits out, the weights once)."""
    from indecis_amd import heads as hd
    rng = np.random.default_rng(11)
    rows = hd.span_tag_count(4)
    w, b = hd.random_head(rows, cfg.hidden, rng)
    model.set_heads([(w, b, True)])
    N = sum(len(s) for s in seqs)
    model.encode_heads(seqs, mean=True, pooled=False)  # warm-up: workspaces
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.encode_heads(seqs, mean=True, pooled=False)
    dt = (time.perf_counter() - t0) / args.steps
    # the head kernel alone: the batch as one part, so that no kernel of
    # another part shares the CUs while its launches are timed
    model.set_option("parts", 1)
    model.encode_heads(seqs, mean=True, pooled=False)
    model.set_profiling(True, only="head_tokens")
    for _ in range(args.steps):
        model.encode_heads(seqs, mean=True, pooled=False)
    st = model.profile()["head_tokens"]
    model.set_profiling(False)
    avg_s = st["ms"] / st["launches"] / 1e3
    per_launch = st["bytes"] / st["launches"]
    gbs = per_launch / avg_s / 1e9
    line = {
        "metric": "spans head logits on every token, with the encoder pass (host ids in, host logits out)",
        "value": round(N / dt, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "ms_per_call": round(dt * 1e3, 3), "higher_is_better": True, "dtype": "int8 encoder, f64 head sums",
        "data": "synthetic",
        "config": {"workload": args.workload, "tokens": N, "sequences": len(seqs), "hidden": cfg.hidden,
                   "head_rows": rows},
        "head_kernel": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                        "frac": round(gbs * 1e9 / PEAK_HBM, 4), "avg_launch_us": round(avg_s * 1e6, 2),
                        "launches_timed": st["launches"], "algorithmic_bytes_per_launch": per_launch},
    }
    print(json.dumps(line), flush=True)


def decide(np, model, cfg, args):
    """DecideInputs-shaped load (model.go:316-330, spans.go:369-383): many
    short inputs, each through the encoder and three pooled-row heads
    (Choice-8, Noul, a 5-option Score: 8 + 1 + 4 logits). Three ways:
      reference: sorted by length, sequential passes of 32 sequences
        (forEachPooled's batchSize, model.go:391-417), pooled rows to the
        host, head.logits there in float64 (heads.go:63-74);
      heads_32: the same passes with the heads on the device
        (ixh_encode_heads), only the logits leaving the GPU;
      heads_all: every input in one ixh_encode_heads call (the library cuts
        passes of at most pass_tokens tokens).
    Host ids in, host logits out; the logits of the three are checked equal
    (the device and host sums are in the same order)."""
    from indecis_amd import heads as hd
    rng = np.random.default_rng(7)
    n = args.inputs
    lens = rng.integers(args.decide_lo, args.decide_hi + 1, size=n)
    seqs = [rng.integers(0, cfg.vocab, size=int(k), dtype=np.int32) for k in lens]
    heads = []
    for rows in (8, 1, 4):
        w, b = hd.random_head(rows, cfg.hidden, rng)
        heads.append((w, rng.standard_normal(rows).astype(np.float32), False))
    model.set_heads(heads)
    W = np.concatenate([h[0] for h in heads]).astype(np.float64)
    bias = np.concatenate([h[1] for h in heads]).astype(np.float64)
    order = sorted(range(n), key=lambda i: len(seqs[i]))
    ntok = int(lens.sum())

    def reference():
        z = np.zeros((n, W.shape[0]))
        for s0 in range(0, n, 32):
            idx = order[s0:s0 + 32]
            pooled = model.encode_seqs([seqs[i] for i in idx]).astype(np.float64)
            z[idx] = pooled @ W.T + bias
        return z

    def heads_32():
        z = np.zeros((n, W.shape[0]))
        for s0 in range(0, n, 32):
            idx = order[s0:s0 + 32]
            zp, _ = model.encode_heads([seqs[i] for i in idx], tokens=False)
            z[idx] = zp
        return z

    def heads_all():
        zp, _ = model.encode_heads([seqs[i] for i in order], tokens=False)
        z = np.zeros((n, W.shape[0]))
        z[order] = zp
        return z

    res = {}
    outs = {}
    for name, fn in (("reference", reference), ("heads_32", heads_32), ("heads_all", heads_all)):
        fn()  # warm-up: workspaces of these shapes
        t0 = time.perf_counter()
        for _ in range(args.steps):
            outs[name] = fn()
        dt = (time.perf_counter() - t0) / args.steps
        res[name] = {"inputs_per_s": round(n / dt, 1), "tokens_per_s": round(ntok / dt, 1),
                     "ms_per_call": round(dt * 1e3, 3)}
    same = (np.array_equal(outs["heads_32"], outs["heads_all"]) and
            np.allclose(outs["reference"], outs["heads_all"], rtol=1e-9, atol=1e-12))
    print(json.dumps({
        "metric": "decision-path inputs/s (DecideInputs: encoder + pooled-row heads)",
        "value": res["heads_all"]["inputs_per_s"], "unit": "inputs/s", "higher_is_better": True,
        "n_gpus": 1, "steps": args.steps, "data": "synthetic",
        "config": {"workload": f"{n} inputs of U[{args.decide_lo},{args.decide_hi}] tokens, base shape, "
                               "Choice-8 + Noul + Score-5 heads", "tokens": ntok},
        "modes": res, "logits_agree": bool(same),
        "speedup_vs_reference_shape": round(res["heads_all"]["inputs_per_s"] / res["reference"]["inputs_per_s"], 2),
    }), flush=True)


def tokenize(np, args):
    """Host tokenizer throughput (tokenizer.go's EncodeMax on many texts):
    ixh_tokenizer_encode_batch on the box's CPU share, beside Hugging Face
    tokenizers (the library whose output the reference reproduces) on the
    same texts and threads, ids checked equal; then text to pooled rows on
    the GPU for one batch, tokenizer included. Texts: documents of
    U[256, 2048] bytes built from the texts of the reference's siglip2-tiny
    fixtures (multilingual, emoji, code), on its tokenizer.json."""
    gold = os.path.join(ROOT, "tests", "golden", "tokenizer")
    pool = [json.loads(line)["text"] for line in open(os.path.join(gold, "tokenizer_cases.jsonl"), encoding="utf-8")]
    pool = [t for t in pool if t]
    rng = np.random.default_rng(11)
    docs = []
    for _ in range(args.docs):
        want, parts, n = int(rng.integers(256, 2049)), [], 0
        while n < want:
            t = pool[int(rng.integers(len(pool)))]
            parts.append(t)
            n += len(t.encode("utf-8")) + 1
        docs.append(" ".join(parts))
    nbytes = sum(len(d.encode("utf-8")) for d in docs)
    threads = min(16, os.cpu_count() or 1)
    os.environ.setdefault("RAYON_NUM_THREADS", str(threads))
    from indecis_amd.tokenizer import Tokenizer
    path = os.path.join(gold, "tokenizer.json")
    tok = Tokenizer(path)

    def rate(fn, reps):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            r = fn()
        return (time.perf_counter() - t0) / reps, r

    native = {}
    for th in (1, threads):
        dt, (ids, offs) = rate(lambda: tok.encode_batch(docs, threads=th), args.steps)
        native[th] = dt
    ntok = int(offs[-1])
    hf = None
    try:
        from tokenizers import Tokenizer as HF
    except ImportError:
        HF = None
    if HF is not None:
        h = HF.from_file(path)
        dt, enc = rate(lambda: h.encode_batch(docs), max(1, args.steps // 2))
        same = all(e.ids == ids[offs[i]:offs[i + 1]].tolist() for i, e in enumerate(enc))
        hf = {"value": round(ntok / dt, 1), "unit": "tokens/s", "threads": threads, "ids_equal": same,
              "kind": "tokenizers (Rust), encode_batch"}
    e2e = None
    # No torch here: with this library loaded before torch (the tokenizer
    # loads it), its HIP runtime found no device once torch had initialised
    # its own; the other modes import torch before loading the library.
    from indecis_amd import _lib
    try:
        gpus = _lib.device_count()
    except _lib.IxhError:
        gpus = 0
    if gpus:
        from indecis_amd.modernbert import BASE, Model, Weights
        model = Model(Weights.random(BASE, seed=4), device=0, lanes=args.lanes)
        batch = docs[:256]

        def text_to_rows():
            i, o = tok.encode_batch(batch, max_len=512, threads=threads)
            return model.encode_seqs([i[o[k]:o[k + 1]] for k in range(len(batch))])
        bi, bo = tok.encode_batch(batch, max_len=512, threads=threads)
        seqs = [bi[bo[k]:bo[k + 1]] for k in range(len(batch))]
        t_all, _ = rate(text_to_rows, args.steps)
        t_enc, _ = rate(lambda: model.encode_seqs(seqs), args.steps)
        t_emb, _ = rate(lambda: model.embed(tok, batch, max_len=512, threads=threads), args.steps)
        model.close()
        e2e = {"texts": len(batch), "tokens": int(bo[-1]), "ms_text_to_rows": round(t_all * 1e3, 3),
               "ms_ids_to_rows": round(t_enc * 1e3, 3), "ms_embed": round(t_emb * 1e3, 3),
               "embed_texts_per_s": round(len(batch) / t_emb, 1),
               "note": "EncodeMax(512) of 256 documents on the host, then EncodeSeqs (host ids in, pooled rows "
                       "out) on the GPU, ModernBERT-base shape"}
    print(json.dumps({
        "metric": "host tokenizer tokens/s (EncodeMax over a batch of documents)",
        "value": round(ntok / native[threads], 1), "unit": "tokens/s", "higher_is_better": True,
        "threads": threads, "data": "synthetic",
        "config": {"workload": f"{len(docs)} documents of U[256,2048] bytes from the siglip2-tiny fixture texts",
                   "tokenizer": "siglip2-tiny tokenizer.json (raw Gemma pipeline, 3,252 ids)",
                   "bytes": nbytes, "tokens": ntok},
        "single_thread": {"value": round(ntok / native[1], 1), "MB_per_s": round(nbytes / native[1] / 1e6, 2)},
        "MB_per_s": round(nbytes / native[threads] / 1e6, 2),
        "hf_tokenizers": hf,
        "text_to_rows": e2e,
    }), flush=True)


def vendor_gemm(args):
    """The vendor int8 GEMM on the encoder's GEMM shapes, for reference:
    torch._int_mm (hipBLASLt) with a plain int32 output, and the same
    shapes in bf16 (torch.matmul), M = the cfg4 batch's 73,621 tokens.
    These do only the GEMM; the library's kernels also dequantise, apply
    the epilogues, the residual, the LayerNorm and the quantisation."""
    import torch
    torch.cuda.set_device(0)
    M = 73621
    res = {}
    for K, N, name in ((768, 2304, "qkv, wi"), (768, 768, "wo"), (1152, 768, "womlp")):
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda")
        b = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda").t()
        a16 = torch.randn(M, K, dtype=torch.bfloat16, device="cuda")
        b16 = torch.randn(N, K, dtype=torch.bfloat16, device="cuda").t().contiguous()
        for label, fn, peak in (("int8", lambda: torch._int_mm(a, b), PEAK_INT8_OPS),
                                ("bf16", lambda: a16 @ b16, 2.5e15)):
            for _ in range(args.warmup):
                fn()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(args.steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / args.steps
            ops = 2.0 * M * N * K
            res[f"{name} K{K} N{N} {label}"] = {"us": round(us, 1), "T_per_s": round(ops / us / 1e6, 1),
                                                "frac_of_dense_peak": round(ops / (us / 1e6) / peak, 4)}
    print(json.dumps({"vendor_gemm": res, "M": M, "steps": args.steps, "int8_peak": PEAK_INT8_OPS,
                      "bf16_peak": 2.5e15}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="cfg4", choices=sorted(WORKLOADS))
    ap.add_argument("--lanes", type=int, default=8)
    ap.add_argument("--cpu-tokens", type=int, default=32768,
                    help="tokens of the batch timed on the CPU baseline (0: skip)")
    ap.add_argument("--parts", type=int, default=0,
                    help="run every phase with the batch in this many parts (profiling runs: 1)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one device copy of 512 MiB (PMC calibration)")
    ap.add_argument("--serving", action="store_true",
                    help="instead: concurrent single-sequence requests, direct calls vs the batcher")
    ap.add_argument("--clients", type=int, default=32)
    ap.add_argument("--requests", type=int, default=40, help="requests per client (--serving)")
    ap.add_argument("--tokenize", action="store_true",
                    help="instead: host tokenizer throughput, and text to pooled rows for one batch")
    ap.add_argument("--docs", type=int, default=4096, help="documents (--tokenize)")
    ap.add_argument("--spans", action="store_true",
                    help="instead: the workload's token-level spans head (9 logits a token) in the pass")
    ap.add_argument("--decide", action="store_true",
                    help="instead: a DecideInputs-shaped load, 32-sequence passes vs heads on the device")
    ap.add_argument("--inputs", type=int, default=8192, help="inputs (--decide)")
    ap.add_argument("--decide-lo", type=int, default=8)
    ap.add_argument("--decide-hi", type=int, default=256)
    ap.add_argument("--option", action="append", default=[], metavar="NAME=VALUE",
                    help="a model option (ixh_model_set_option) for every pass, e.g. fuse_mlp=2")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="instead: the vendor int8 and bf16 GEMMs (torch) on the encoder's GEMM shapes")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {max(args.gpus, world)}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    if args.vendor_gemm:
        vendor_gemm(args)
        return
    import numpy as np
    if args.tokenize:
        tokenize(np, args)
        return
    import torch

    from indecis_amd import _lib
    from indecis_amd.modernbert import BASE, SMALL, Model, Weights

    mname, B, lo, hi = WORKLOADS[args.workload]
    cfg = BASE if mname == "base" else SMALL
    if mname == "bekko":
        from indecis_amd.modernbert import Config
        cfg = Config(hidden=384, layers=22, heads=6, intermediate=1152, vocab=32768)
    weights = Weights.random(cfg, seed=4)
    seqs = make_inputs(np, cfg.vocab, B, lo, hi)
    offs = np.zeros(B + 1, np.int32)
    offs[1:] = np.cumsum([len(s) for s in seqs])
    N = int(offs[-1])

    torch.cuda.set_device(0)
    model = Model(weights, device=0, lanes=args.lanes)
    for o in args.option:
        k, v = o.split("=", 1)
        model.set_option(k, int(v))
    if args.serving:
        serving(np, model, cfg, args)
        model.close()
        return
    if args.decide:
        decide(np, model, cfg, args)
        model.close()
        return
    if args.spans:
        spans(np, model, cfg, seqs, args)
        model.close()
        return
    ids_d = torch.from_numpy(np.concatenate(seqs)).to("cuda")
    out_d = torch.empty((B, cfg.hidden), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        model.encode_device(ids_d.data_ptr(), offs, out_d.data_ptr(), _lib.OUT_POOLED, stream)

    if args.parts:
        model.set_option("parts", args.parts)  # warm-up passes shaped as the measured ones
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    if args.copy_probe:
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # One untimed pass, the batch as one part (no concurrent kernels), with
    # every launch bracketed by events: the per-class breakdown and the
    # dominant class.
    model.set_option("parts", args.parts or 1)
    model.set_profiling(True)
    step()
    torch.cuda.synchronize()
    breakdown = model.profile()
    dom = max(breakdown, key=lambda k: breakdown[k]["ms"])

    def timed(parts):
        """K timed steps with the batch in `parts` parts (0 = the library's
        default split); events around the dominant class's launches only
        (two per launch, on the stream each runs on)."""
        model.set_option("parts", args.parts or parts)
        step()  # untimed: workspaces of this split
        model.set_profiling(True, only=dom)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        st = model.profile()[dom]
        model.set_profiling(False)
        return wall * 1000 / args.steps, e0.elapsed_time(e1) / args.steps, st

    # Headline: the library's default (a large batch runs as parts on
    # several streams). Roofline: the dominant class running alone.
    ms_per_step, gpu_ms, d_conc = timed(0)
    ms_alone, _, d = timed(1)
    model.set_option("parts", 0)

    # per-class figures of the untimed pass (one step)
    kernels = {}
    for name, st in breakdown.items():
        per_launch_ms = st["ms"] / max(st["launches"], 1)
        if st["ops"] > 0:
            ach = st["ops"] / (st["ms"] / 1e3) / 1e12
            kernels[name] = {"ms_per_step": round(st["ms"], 3), "TOP/s": round(ach, 1),
                             "mfma_frac": round(ach * 1e12 / PEAK_INT8_OPS, 4)}
        else:
            ach = st["bytes"] / (st["ms"] / 1e3) / 1e9
            kernels[name] = {"ms_per_step": round(st["ms"], 3), "GB/s": round(ach, 1),
                             "hbm_frac": round(ach * 1e9 / PEAK_HBM, 4)}
        kernels[name]["avg_launch_us"] = round(per_launch_ms * 1e3, 2)
    avg_s = d["ms"] / d["launches"] / 1e3
    if d["ops"] > 0:
        per_launch = d["ops"] / d["launches"]
        roof = {"bound": "mfma", "achieved": round(per_launch / avg_s / 1e12, 2),
                "peak": PEAK_INT8_OPS / 1e12, "unit": "TOP/s"}
    else:
        per_launch = d["bytes"] / d["launches"]
        roof = {"bound": "hbm", "achieved": round(per_launch / avg_s / 1e9, 1),
                "peak": PEAK_HBM / 1e9, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = load_traffic(dom, args.workload)
    roof["kernel"] = dom
    roof["algorithmic_per_launch"] = per_launch
    roof["avg_launch_us"] = round(avg_s * 1e6, 2)
    roof["launches_timed"] = d["launches"]
    roof["note"] = (f"dominant class running alone: {args.steps} more timed steps with the batch as one part "
                    f"({ms_alone:.3f} ms/step)")
    c_avg = d_conc["ms"] / d_conc["launches"] / 1e3
    c_per = (d_conc["ops"] or d_conc["bytes"]) / d_conc["launches"]
    roof_conc = {"achieved": round(c_per / c_avg / (1e12 if d_conc["ops"] else 1e9), 2 if d_conc["ops"] else 1),
                 "unit": roof["unit"], "launches": d_conc["launches"], "avg_launch_us": round(c_avg * 1e6, 2),
                 "note": "same class inside the headline timed region, where the parts' kernels overlap"}
    roof_conc["frac"] = round(roof_conc["achieved"] / roof["peak"], 4)
    # the GEMM-bearing classes: the GEMM kernels and the fused MLP block
    gemm = [st for n, st in breakdown.items() if n.startswith("gemm_") or n == "mlp_ln"]
    gemm_ops = sum(st["ops"] for st in gemm)
    gemm_ms = sum(st["ms"] for st in gemm)

    # the device's own int8 MFMA rate (every wave issuing MFMAs from
    # registers): the scale the kernels' fractions of the dense peak sit on
    from indecis_amd import linalg
    loop_rate = linalg.check_mfma_rate(0)

    cpu = None
    if args.cpu_tokens > 0:
        cpu = cpu_baseline(np, weights, seqs, args.cpu_tokens)

    line = {
        "metric": "encoder tokens/sec (int8, 512-tok, batch 256) + % of int8 MFMA peak",
        "value": round(N / (ms_per_step / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "gpu_ms_per_step": round(gpu_ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: ModernBERT-{mname}-shaped int8 encoder, "
                               f"batch {B} x U[{lo},{hi}] tokens packed by offsets, random-init",
                   "tokens_per_step": N, "sequences": B, "hidden": cfg.hidden,
                   "layers": cfg.layers, "heads": cfg.heads, "intermediate": cfg.intermediate,
                   "vocab": cfg.vocab, "lanes": args.lanes, "parallelism": "single GPU"},
        "seqs_per_s": round(B / (ms_per_step / 1e3), 1),
        "gemm_mfma_frac": round(gemm_ops / (gemm_ms / 1e3) / PEAK_INT8_OPS, 4) if gemm_ms else None,
        "roofline": roof,
        "roofline_concurrent": roof_conc,
        "mfma_loop": {"TOP/s": round(loop_rate / 1e12, 1), "frac": round(loop_rate / PEAK_INT8_OPS, 4),
                      "note": "int8 MFMAs issued back to back from registers by four waves a SIMD "
                              "(ixh_check_mfma_rate), after the timed region"},
        "cpu_baseline": cpu,
        "kernels": kernels,
        "kernels_note": "per kernel class, from one untimed pass with every launch timed by HIP events",
    }
    print(json.dumps(line), flush=True)
    model.close()


if __name__ == "__main__":
    main()
