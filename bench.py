#!/usr/bin/env python3
"""Benchmark: accepted tokens/sec of the speculative decoding loop at 7B shape.

Workload: random-init (synthetic) Llama target -- dim 4096, 32 layers, 32
heads, FFN 11008, vocab 32000 -- and draft -- dim 2048, 16 layers, 16 heads,
FFN 5632 -- all linear layers, the embedding and the LM head GGUF Q4_K; a
seeded prompt of 2048 tokens (prefill untimed); k = 5 draft tokens per step;
batch 1 (--batch B: B sequences of their own 2048-token prompts stepped
together, the target verifying 6 B rows per step); temperature 0.8 over the
full vocabulary (--greedy: argmax rule).  One step = 5 draft forwards + one
target forward over 6 rows per sequence + acceptance + commit, replayed from a
captured HIP graph.  Inputs live in HBM before the timed region starts.

Printed (one JSON line): value = committed tokens / wall seconds over exactly
--steps steps, bracketed by stream synchronisations; "roofline" for the verify
dequant-GEMM (the dominant kernel): algorithmic bytes of the target's 129
verify GEMMs at M = 6 over their average duration, measured with HIP events
on the context stream; "cpu_baseline": the CPU restatement timed on the host
on the first recorded steps (from the GPU's post-prefill KV cache), with the
step-by-step parity of the draws and accept decisions.
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO, "universal-loader_amd")

TARGET = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=32, ffn=11008, vocab=32000, rms_eps=1e-5,
              rope_base=10000.0)
DRAFT = dict(dim=2048, n_layers=16, n_heads=16, n_kv_heads=16, ffn=5632, vocab=32000, rms_eps=1e-5,
             rope_base=10000.0)
CONTEXT = 2048
K_SPEC = 5
HBM_PEAK_GBS = 8000.0
METRIC = "accepted tokens/sec, 7B-shape Q4_K k=5 bs=1; verify-GEMM HBM GB/s % of peak"


def load_package():
    spec = importlib.util.spec_from_file_location("universal_loader_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["universal_loader_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_ids(pkg, ctx):
    """Ids and (type, N, K) of every weight on the context, in creation order."""
    out = []
    while True:
        try:
            out.append((len(out), ctx.weight_info(len(out))))
        except pkg.UlspecError:
            return out


def gemm_roofline(pkg, ctx, ids, M, reps=10):
    """Average duration and algorithmic bytes of the verify GEMM over the given
    weights at M rows: reps rounds of back-to-back launches over all weights
    (direct launches, so that a profiler sees every dispatch), HIP events on
    the context stream around them."""
    kmax = max(info[2] for _, info in ids)
    nmax = max(info[1] for _, info in ids)
    rng = np.random.default_rng(0)
    x = ctx.upload(rng.standard_normal((M, kmax)).astype(np.float16).view(np.uint16))
    y = ctx.alloc(M * nmax * 4)
    for wid, _ in ids:  # warm-up round
        ctx.verify_gemm(wid, x, M, y)
    ctx.sync()
    ctx.timer_mark(2)
    for _ in range(reps):
        for wid, _ in ids:
            ctx.verify_gemm(wid, x, M, y)
    ctx.timer_mark(3)
    ms = ctx.timer_elapsed_ms(2, 3)
    x.free()
    y.free()
    launches = reps * len(ids)
    alg = 0.0
    for _, (wtype, n, k, _) in ids:
        w_bytes = n * k * (144 / 256 if wtype == pkg.Q4_K else 18 / 32)
        alg += w_bytes + 2 * M * k + 4 * M * n
    us = ms * 1e3 / launches
    return us, alg / len(ids)


def instep_gemm_roofline(pkg, model, ids, M, pos, reps=10):
    """The target's verify GEMMs as a speculative step runs them: every layer's
    Q|K|V, O, gate|up and down linear plus the LM head, each with its fused
    prologue and epilogue (split fp16 X operands, RMSNorm row scale, RoPE + K/V
    append, SiLU, residual), M rows at position pos, launched alone
    (ulspec_model_linear, direct launches) on the activations the model's last
    forward left; reps rounds back to back, HIP events on the context stream
    around them.  Average us per GEMM call (the split-K down projection's
    reduction launch included) and algorithmic bytes per call."""
    ctx = model.ctx
    L = model.cfg.n_layers
    calls = [(l, w) for l in range(L) for w in range(4)] + [(0, model.LIN_HEAD)]

    def one_round():
        for l, w in calls:
            model.linear(l, w, M, pos)
    one_round()  # warm-up
    ctx.sync()
    ctx.timer_mark(2)
    for _ in range(reps):
        one_round()
    ctx.timer_mark(3)
    ms = ctx.timer_elapsed_ms(2, 3)
    alg = 0.0
    for _, (wtype, n, k, _) in ids:
        alg += n * k * (144 / 256 if wtype == pkg.Q4_K else 18 / 32) + 2 * M * k + 4 * M * n
    assert len(ids) == len(calls)
    return ms * 1e3 / (reps * len(calls)), alg / len(ids)


def read_traffic():
    """HBM bytes per call of the in-step verify GEMMs from the committed PMC
    summary (FETCH_SIZE + WRITE_SIZE, calibrated), or None."""
    path = os.path.join(REPO, "profiles", "verify_gemm_q4k_7b_m6_instep_pmc.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch"):
                    return float(line.split("=")[1])
    except OSError:
        pass
    return None


def cpu_leg(pkg, args, target_host, draft_host, kv_t, kv_d, recorded, seq, cap, n0):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as ora
    nproc, allowed, nt = ora.host_cpus()
    s = ora.sampling(greedy=True) if args.greedy else ora.sampling(temperature=args.temperature)
    models = []
    for cfg, host, kv in ((TARGET, target_host, kv_t), (DRAFT, draft_host, kv_d)):
        m = ora.Llama(**cfg, max_ctx=cap, nthreads=nt)
        for name, (wtype, data, ne0, ne1) in host.items():
            m.set_tensor(name, wtype, data, ne0, ne1)
        for l, (k, v) in enumerate(kv):
            m.kv_io(l, 1, 0, n0 - 1, k, v)
        models.append(m)
    ot, od = models
    k = K_SPEC
    busy = 0.0
    steps = tokens = 0
    draws_exact = accept_exact = own_agree = True
    worst = 0.0
    def cpu_step(n, r, threads):
        """The CPU path's own step on the GPU's committed and draft tokens."""
        d, u = r["draft_tokens"], r["uniforms"]
        dl = [od.forward(seq[n - 2:n], n - 2, n_logits=1)[0]]
        own_d = [ora.sample(s, dl[0][None], u[0:1])[0]]
        for j in range(1, k):
            dl.append(od.forward(d[j - 1:j], n - 1 + j, n_logits=1)[0])
            own_d.append(ora.sample(s, dl[j][None], u[j:j + 1])[0])
        dl = np.array(dl)
        tl = ot.forward(np.concatenate([[seq[n - 1]], d]).astype(np.int32), n - 1, n_logits=k + 1)
        out_c, nacc_c = ora.accept(s, tl[None], dl[None], d[None], u[k:][None], nthreads=threads)
        return dl, own_d, tl, nacc_c

    for n, r in recorded:
        if busy > args.cpu_seconds:
            break
        d, u = r["draft_tokens"], r["uniforms"]
        t0 = time.perf_counter()
        dl, own_d, tl, nacc_c = cpu_step(n, r, nt)
        busy += time.perf_counter() - t0
        steps += 1
        tokens += int(nacc_c[0]) + 1
        # parity against the GPU step (checker, untimed)
        for j in range(k):
            draws_exact &= bool(ora.sample(s, r["draft_logits"][j:j + 1], u[j:j + 1])[0] == d[j])
        out_g, nacc_g = ora.accept(s, r["target_logits"][None], r["draft_logits"][None], d[None], u[k:][None])
        accept_exact &= bool(int(nacc_g[0]) == r["n_accepted"] and np.array_equal(out_g[0], r["out_tokens"]))
        own_agree &= bool(int(nacc_c[0]) == r["n_accepted"] and list(own_d) == list(d))
        for a, b in ((r["draft_logits"], dl), (r["target_logits"], tl)):
            b64 = b.astype(np.float64)
            worst = max(worst, float(np.abs(a - b64).max() / np.sqrt((b64 ** 2).mean())))
    # the same steps on one thread (a bounded sample: at least two steps)
    for m in models:
        m.set_threads(1)
    busy1, tokens1, steps1 = 0.0, 0, 0
    for n, r in recorded[:steps]:
        if steps1 >= 2 and busy1 > args.cpu_seconds / 2:
            break
        t0 = time.perf_counter()
        _, _, _, nacc1 = cpu_step(n, r, 1)
        busy1 += time.perf_counter() - t0
        tokens1 += int(nacc1[0]) + 1
        steps1 += 1
    for m in models:
        m.close()
    mode = "greedy" if args.greedy else f"T={args.temperature}"
    return {
        "value": tokens / busy if busy else None, "unit": "tokens/s", "cores": nt, "kind": "port",
        "nproc": nproc, "cpus_allowed": allowed, "threads": nt,
        "value_1thread": tokens1 / busy1 if busy1 else None, "steps_1thread": steps1, "cpu_model": _cpu_model(),
        "sample": f"{steps} speculative steps (k=5, {mode}) of the 7B-shape Q4_K target/draft pair at context "
                  f"{n0}, from the GPU's post-prefill KV cache; oracle/ C restatement, AVX2 f32 GEMM, {nt} threads "
                  f"(value: the CPUs this process may use, {allowed} of nproc {nproc}, capped at the 16-core host "
                  f"share of one GPU), the first {steps1} of them on 1 thread (value_1thread)",
        "parity": {"steps": steps, "draft_draws_bit_exact": draws_exact, "accept_bit_exact": accept_exact,
                   "cpu_decisions_equal_gpu": own_agree, "logits_max_err_over_rms": worst},
    }


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _ora():
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    return oracle


def _copies(nbytes, total=600e6):
    """Copies of an input of nbytes that rotate through more than the 256 MB
    last-level cache (at least 2)."""
    return max(2, int(np.ceil(total / nbytes)))


def _time_direct(ctx, fn, reps):
    """Average us per call of fn() over reps back-to-back direct launches (HIP
    events on the context stream)."""
    fn()
    ctx.sync()
    ctx.timer_mark(4)
    for _ in range(reps):
        fn()
    ctx.timer_mark(5)
    return ctx.timer_elapsed_ms(4, 5) * 1e3 / reps


def workload_gemm(pkg, ctx, args):
    """Verify dequant-GEMM alone: Q4_0 weights N(0, 0.02^2), fp16 X N(0,1),
    M in {1,5,9,17}; 24 copies of each weight rotated (> 256 MB, past the
    MALL).  Headline: N=4096, K=11008, M=5."""
    ora = _ora()
    rng = np.random.default_rng(args.seed)
    rows, head = [], None
    for N, K in ((4096, 4096), (11008, 4096), (4096, 11008)):
        nb = N * pkg.row_bytes(pkg.Q4_0, K)
        buf = ctx.alloc(nb)
        ctx.synth_q4(pkg.Q4_0, 7, N + K, N, K, 0.02, buf)
        W = ctx.download(buf, np.uint8, (nb,))
        buf.free()
        ids = [ctx.weight_upload(pkg.Q4_0, W, N, K) for _ in range(24)]
        for M in (1, 5, 9, 17):
            X = rng.standard_normal((M, K)).astype(np.float16).view(np.uint16)
            xb, yb = ctx.upload(X), ctx.alloc(M * N * 4)
            it = iter(range(1 << 30))
            us = _time_direct(ctx, lambda: ctx.verify_gemm(ids[next(it) % 24], xb, M, yb), 24 * args.reps)
            alg = nb + 2 * M * K + 4 * M * N
            gbs = alg / us / 1e3
            rows.append({"N": N, "K": K, "M": M, "us": us, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS})
            log(f"Q4_0 N={N} K={K} M={M}: {us:.2f} us, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s)")
            if (N, K, M) == (4096, 11008, 5):
                head = (us, alg, gbs)
                Y = ctx.download(yb, np.float32, (M, N))
                ref = ora.q4_gemm_f64(pkg.Q4_0, W, N, K, X)
                err = float(np.abs(Y - ref).max() / np.sqrt((ref ** 2).mean()))
                # CPU baseline: the oracle's AVX2 f32 dequant-GEMM on the same inputs
                t0, n = time.perf_counter(), 0
                while time.perf_counter() - t0 < args.cpu_seconds:
                    ora.q4_gemm_f32(pkg.Q4_0, W, N, K, X)
                    n += 1
                cpu_gbs = alg * n / (time.perf_counter() - t0) / 1e9
            xb.free()
            yb.free()
    us, alg, gbs = head
    return {
        "metric": "verify-GEMM HBM GB/s (Q4_0 4096x11008, M=5)", "value": gbs, "unit": "GB/s", "ms_per_step": us / 1e3,
        "dtype": "q4_0 weights x fp16 activations, fp32 accumulate",
        "config": {"workload": "Q4_0 verify dequant-GEMM N=4096 K=11008 M=5, 24 rotated weight copies", "table": rows},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": None, "avg_us": us, "algorithmic_bytes": alg},
        "cpu_baseline": {"value": cpu_gbs, "unit": "GB/s", "cores": ora.nthreads_default(), "kind": "port",
                         "sample": "oracle AVX2 f32 dequant-GEMM, N=4096 K=11008 M=5, repeated "
                                   f"for {args.cpu_seconds:.0f} s"},
        "parity": {"max_err_over_rms_vs_f64": err},
    }


def workload_attention(pkg, ctx, args):
    """Verify attention alone: 32 heads x 128, fp16 K/V of 4096 prior tokens
    N(0,1); 5 causal queries and a 16-node draft tree (branching <= 3, depth
    <= 5).  Headline: the causal case."""
    ora = _ora()
    rng = np.random.default_rng(args.seed)
    H, D, P = 32, 128, 4096
    out, head = [], None
    parents = {"causal5": None, "tree16": np.array([-1, 0, 0, 1, 1, 2, 3, 3, 4, -1, 9, 9, 10, 5, 13, 6], np.int32)}
    for name, parent in parents.items():
        nq = 5 if parent is None else 16
        L = P + nq
        q = rng.standard_normal((nq, H, D)).astype(np.float16).view(np.uint16)
        k = rng.standard_normal((L, H, D)).astype(np.float16).view(np.uint16)
        v = rng.standard_normal((L, H, D)).astype(np.float16).view(np.uint16)
        alg = 2 * L * H * D * 2 + nq * H * D * (2 + 4)
        nc = _copies(alg)
        bq, bo = ctx.upload(q), ctx.alloc(nq * H * D * 4)
        kv = [(ctx.upload(k), ctx.upload(v)) for _ in range(nc)]
        bk, bv = kv[0]
        scale = 1.0 / np.sqrt(D)
        it = iter(range(1 << 30))

        def call():
            ck, cv = kv[next(it) % nc]
            ctx.verify_attention(bq, ck, cv, P, nq, parent, H, H, D, scale, bo)
        us = _time_direct(ctx, call, nc * args.reps)
        ctx.verify_attention(bq, bk, bv, P, nq, parent, H, H, D, scale, bo)
        gbs = alg / us / 1e3
        o = ctx.download(bo, np.float32, (nq, H, D))
        ref = ora.attention_f64(q, k, v, P, parent, H, H, D, scale)
        err = float(np.abs(o - ref).max())
        out.append({"case": name, "us": us, "GB/s": gbs, "max_abs_err_vs_f64": err, "rotated_copies": nc})
        log(f"attention {name}: {us:.2f} us, {gbs:.0f} GB/s, max err {err:.1e}")
        if name == "causal5":
            head = (us, alg, gbs)
            t0, n = time.perf_counter(), 0
            while time.perf_counter() - t0 < args.cpu_seconds:
                ora.attention_f32(q, k, v, P, None, H, H, D, scale)
                n += 1
            cpu_gbs = alg * n / (time.perf_counter() - t0) / 1e9
        for b in (bq, bo, *[x for pair in kv for x in pair]):
            b.free()
    us, alg, gbs = head
    return {
        "metric": "verify-attention HBM GB/s (32x128, prefix 4096, 5 causal queries)", "value": gbs, "unit": "GB/s",
        "ms_per_step": us / 1e3, "dtype": "fp16 K/V, fp32 softmax",
        "config": {"workload": "verify attention H=32 D=128 prefix 4096, causal nq=5 (and tree nq=16), K/V rotated "
                               "over copies totalling > 512 MB", "cases": out},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": None, "avg_us": us, "algorithmic_bytes": alg},
        "cpu_baseline": {"value": cpu_gbs, "unit": "GB/s", "cores": ora.nthreads_default(), "kind": "port",
                         "sample": f"oracle f32 attention, causal nq=5, repeated for {args.cpu_seconds:.0f} s"},
    }


def workload_accept(pkg, ctx, args):
    """Acceptance sampling alone: B=16 sequences, k in {4, 8}, V in {32000,
    128256}; logits N(0, 3^2) with one +8 boost per row; T 0.8, top-k 40,
    top-p 0.9 (and the greedy rule).  Headline: k=4, V=32000."""
    ora = _ora()
    rng = np.random.default_rng(args.seed)
    B = 16
    cases, head = [], None
    for k, V in ((4, 32000), (8, 32000), (4, 128256), (8, 128256)):
        tl = (3.0 * rng.standard_normal((B, k + 1, V))).astype(np.float32)
        dl = (3.0 * rng.standard_normal((B, k, V))).astype(np.float32)
        for a in (tl, dl):
            flat = a.reshape(-1, V)
            flat[np.arange(flat.shape[0]), rng.integers(0, V, flat.shape[0])] += 8.0
        s_ora = ora.sampling(temperature=0.8, top_k=40, top_p=0.9)
        dt = np.stack([ora.sample(s_ora, dl[b], ora.uniforms(args.seed + 1, b * k, k)) for b in range(B)])
        u = np.stack([ora.uniforms(args.seed + 2, b * (k + 1), k + 1) for b in range(B)])
        nc = _copies(tl.nbytes + dl.nbytes)
        logit_bufs = [(ctx.upload(tl), ctx.upload(dl)) for _ in range(nc)]
        btl, bdl = logit_bufs[0]
        bdt, bu = ctx.upload(dt), ctx.upload(u)
        bo, bn = ctx.alloc(B * (k + 1) * 4), ctx.alloc(B * 4)
        for greedy in (False, True):
            s = pkg.sampling(greedy=True) if greedy else pkg.sampling(temperature=0.8, top_k=40, top_p=0.9)
            it = iter(range(1 << 30))

            def call():
                ct, cd = logit_bufs[next(it) % nc]
                ctx.accept(s, B, k, V, ct, cd, bdt, bu, bo, bn)
            us = _time_direct(ctx, call, nc * args.reps)
            ctx.accept(s, B, k, V, btl, bdl, bdt, bu, bo, bn)
            alg = 4 * B * (2 * k + 1) * V if not greedy else 4 * B * (k + 1) * V
            gbs = alg / us / 1e3
            got = ctx.download(bo, np.int32, (B, k + 1))
            want, _ = ora.accept(ora.sampling(greedy=True) if greedy else s_ora, tl, dl, dt, u)
            exact = bool(np.array_equal(got, want))
            cases.append({"k": k, "V": V, "greedy": greedy, "us": us, "GB/s": gbs, "bit_exact": exact,
                          "rotated_copies": nc})
            log(f"accept k={k} V={V} greedy={greedy}: {us:.2f} us, {gbs:.0f} GB/s, bit-exact {exact}")
            if (k, V, greedy) == (4, 32000, False):
                head = (us, alg, gbs)
                t0, n = time.perf_counter(), 0
                while time.perf_counter() - t0 < args.cpu_seconds:
                    ora.accept(s_ora, tl, dl, dt, u)
                    n += 1
                cpu_gbs = alg * n / (time.perf_counter() - t0) / 1e9
        for b in (bdt, bu, bo, bn, *[x for pair in logit_bufs for x in pair]):
            b.free()
    us, alg, gbs = head
    return {
        "metric": "acceptance-sampling HBM GB/s (B=16, k=4, V=32000)", "value": gbs, "unit": "GB/s",
        "ms_per_step": us / 1e3, "dtype": "fp32 logits, exact u64 fixed point",
        "config": {"workload": "acceptance sampling B=16 k=4 V=32000, T 0.8 top-k 40 top-p 0.9, logits rotated over "
                               "copies totalling > 512 MB", "cases": cases},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": None, "avg_us": us, "algorithmic_bytes": alg},
        "cpu_baseline": {"value": cpu_gbs, "unit": "GB/s", "cores": ora.nthreads_default(), "kind": "port",
                         "sample": f"oracle accept rule, same inputs, repeated for {args.cpu_seconds:.0f} s"},
    }


def workload_q6k(pkg, ctx, args):
    """The LM-head-shaped verify GEMM of Q4_K_M files, output.weight 32000 x
    4096 in Q6_K at M = 6: the native Q6_K kernel (0.82 B per weight) against
    the same shape held as fp16 (2 B per weight, how Q6_K was run before).
    Random Q6_K blocks (every 6-bit value and int8 scale is valid; d = 2^-12)
    and random fp16 weights; copies rotated past the last-level cache."""
    N, K, M = 32000, 4096, 6
    rng = np.random.default_rng(args.seed)
    nsb = K // 256
    X = rng.standard_normal((M, K)).astype(np.float16).view(np.uint16)
    xb, yb = ctx.upload(X), ctx.alloc(M * N * 4)
    rows, out = [], {}
    for name, wtype, nbytes in (("q6_k", pkg.Q6_K, N * nsb * 210), ("f16", pkg.F16, N * K * 2)):
        if wtype == pkg.Q6_K:
            blocks = rng.integers(0, 256, (N, nsb, 210), dtype=np.uint8)
            blocks[:, :, 208:210] = np.full((N, nsb, 1), 2.0 ** -12, np.float16).view(np.uint8)
        else:
            blocks = (rng.standard_normal((N, K)) * 0.02).astype(np.float16).view(np.uint8)
        nc = _copies(nbytes)
        ids = [ctx.weight_upload(wtype, blocks, N, K) for _ in range(nc)]
        del blocks
        it = iter(range(1 << 30))
        us = _time_direct(ctx, lambda: ctx.verify_gemm(ids[next(it) % nc], xb, M, yb), nc * args.reps)
        alg = nbytes + 2 * M * K + 4 * M * N
        gbs = alg / us / 1e3
        out[name] = (us, alg, gbs)
        rows.append({"type": name, "bytes_per_weight": nbytes / (N * K), "us": us, "GB/s": gbs,
                     "weights_per_us": N * K / us})
        log(f"{name} N={N} K={K} M={M}: {us:.2f} us, {alg / 1e6:.1f} MB, {gbs:.0f} GB/s "
            f"({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s), {N * K / us / 1e6:.2f} G weights/ms")
    xb.free()
    yb.free()
    us, alg, gbs = out["q6_k"]
    return {
        "metric": "Q6_K verify-GEMM HBM GB/s (32000x4096, M=6)", "value": gbs, "unit": "GB/s", "ms_per_step": us / 1e3,
        "dtype": "q6_k weights x fp16 activations, fp32 accumulate",
        "config": {"workload": "Q6_K verify dequant-GEMM N=32000 K=4096 M=6 against the fp16-held weight",
                   "table": rows, "speedup_vs_f16": out["f16"][0] / us},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": None, "avg_us": us, "algorithmic_bytes": alg},
        "cpu_baseline": None,
    }


# Weight bytes of the 7B-shape step's linears (Q4_K: 144 B per 256 weights)
STEP_WEIGHTS = (("draft O", 2359296), ("draft down", 6488064), ("draft QKV", 7077888), ("target O", 9437184),
                ("draft gate/up", 12976128), ("target down", 25362432), ("target QKV", 28311552),
                ("target gate/up", 50724864))


def workload_read(pkg, ctx, args):
    """Streaming-read ceiling: the plain 16-byte-load read kernel over the
    byte counts of the verify GEMMs (the Q4_0 4096x11008 weight, the 7B Q4_K
    QKV and gate/up weights), 24 rotated copies of each (> 512 MB, past the
    MALL), every load variant, direct launches; the fastest variant per size
    is the ceiling.  Variants 4..7 repeat 0..3 with non-temporal loads (the
    cache policy the verify GEMMs read their weights with).  Then the same
    reads at the weight sizes of every linear of the 7B-shape step, 48
    launches over 24 copies captured in a HIP graph and replayed (the setting
    the step runs in): the per-launch floor of a GEMM that reads those
    bytes."""
    sink = ctx.alloc(16)
    rows, head = [], None
    for nbytes in (25362432, 28311552, 50724864):
        bufs = [ctx.alloc(nbytes) for _ in range(24)]  # contents do not matter (the XOR only feeds the sink test)
        best = None
        for variant in range(8):
            it = iter(range(1 << 30))
            us = _time_direct(ctx, lambda: ctx.stream_read(bufs[next(it) % 24], nbytes, variant, sink),
                              24 * args.reps)
            gbs = nbytes / us / 1e3
            nt = variant >= 4
            log(f"read {nbytes / 1e6:.1f} MB, {4 << (variant & 3)} loads per thread{' non-temporal' if nt else ''}: "
                f"{us:.2f} us, {gbs:.0f} GB/s")
            rows.append({"bytes": nbytes, "loads_per_thread": 4 << (variant & 3), "non_temporal": nt, "us": us,
                         "GB/s": gbs})
            if best is None or us < best[0]:
                best = (us, gbs, variant)
        if nbytes == 25362432:
            head = best
        for b in bufs:
            b.free()
    graph_rows = []
    for name, nbytes in STEP_WEIGHTS:
        bufs = [ctx.alloc(nbytes) for _ in range(24)]
        per = []
        for variant in range(8):
            ctx.capture_begin()
            for i in range(48):
                ctx.stream_read(bufs[i % 24], nbytes, variant, sink)
            gid = ctx.capture_end()
            ctx.graph_replay(gid, 2)
            ctx.sync()
            ctx.timer_mark(0)
            ctx.graph_replay(gid, args.reps)
            ctx.timer_mark(1)
            ctx.sync()
            per.append(ctx.timer_elapsed_ms(0, 1) * 1e3 / (48 * args.reps))
            ctx.graph_destroy(gid)
        us = min(per)
        log(f"graph-replayed read, {name} weight ({nbytes / 1e6:.2f} MB): " +
            " / ".join(f"{u:.2f}" for u in per) + f" us (4 / 8 / 16 / 32 loads per thread, plain then "
            f"non-temporal), best "
            f"{nbytes / us / 1e3:.0f} GB/s")
        graph_rows.append({"linear": name, "bytes": nbytes, "us_by_variant": per, "best_us": us})
        for b in bufs:
            b.free()
    sink.free()
    us, gbs, variant = head
    return {
        "metric": "streaming-read ceiling GB/s (25.4 MB, the Q4_0 4096x11008 weight)", "value": gbs, "unit": "GB/s",
        "ms_per_step": us / 1e3, "dtype": "u8",
        "config": {"workload": "plain 16-byte-load read of 25 / 28 / 51 MB buffers, 24 rotated copies", "table": rows,
                   "best_loads_per_thread": 4 << (variant & 3), "best_non_temporal": variant >= 4,
                   "graph_replayed_step_weights": graph_rows},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": None, "avg_us": us, "algorithmic_bytes": 25362432},
        "cpu_baseline": None,
    }


def workload_launch(pkg, ctx, args):
    """The per-launch floor of a graph-replayed step: 100 back-to-back launches
    of a tiny kernel (the uniforms kernel: one 256-thread workgroup, and 1024
    of them) captured into one HIP graph and replayed, HIP events around the
    replays; against the grid-wide barrier a persistent kernel would use in
    place of a kernel boundary (ulspec_sync_probe: one workgroup per CU, all
    co-resident, 2000 rounds), with agent-scope release / acquire (mode 0) and
    with write-through data and flags (mode 1)."""
    rows = []
    buf = ctx.alloc(256 * 1024 * 4)
    for n in (64, 256 * 1024):
        ctx.capture_begin()
        for _ in range(100):
            ctx.uniforms(1, 0, n, buf)
        gid = ctx.capture_end()
        ctx.graph_replay(gid, 2)
        ctx.sync()
        ctx.timer_mark(0)
        ctx.graph_replay(gid, 20)
        ctx.timer_mark(1)
        ctx.sync()
        us = ctx.timer_elapsed_ms(0, 1) * 1e3 / 2000
        ctx.graph_destroy(gid)
        rows.append({"what": f"graph-replayed launch, {(n + 255) // 256} workgroups of 256", "us": us})
        log(f"graph-replayed launch of {(n + 255) // 256} workgroups: {us:.3f} us")
    buf.free()
    n_cu = ctx.n_cu
    for mode in (0, 1):
        for wg, thr in ((n_cu, 1024), (n_cu, 256), (n_cu // 2, 1024)):
            us, err = ctx.sync_probe(mode, wg, thr, 2000)
            rows.append({"what": f"grid barrier mode {mode}, {wg} x {thr}", "us": us, "stale_reads": err})
            log(f"grid barrier mode {mode}: {wg} workgroups x {thr}: {us:.2f} us per round, {err} stale reads")
    floor = rows[0]["us"]
    return {"metric": "graph-replayed launch floor (us)", "value": floor, "unit": "us", "higher_is_better": False,
            "ms_per_step": floor / 1e3, "dtype": "n/a",
            "config": {"workload": "launch floor against grid-wide barriers", "table": rows},
            "roofline": None, "cpu_baseline": None}


def workload_copy(pkg, ctx, args):
    """Calibration: device-to-device copies of 25362432 bytes (the size of a
    4096 x 11008 Q4_0 weight), the reference point that scales the FETCH_SIZE /
    WRITE_SIZE counters to bytes."""
    nb = 25362432
    a, b = ctx.alloc(nb), ctx.alloc(nb)
    us = _time_direct(ctx, lambda: pkg.lib().ulspec_memcpy(ctx.handle, b.ptr, a.ptr, nb, 2), args.reps)
    a.free()
    b.free()
    gbs = 2 * nb / us / 1e3
    log(f"copy {nb} B: {us:.2f} us, {gbs:.0f} GB/s (read + write)")
    return {"metric": "device copy GB/s (read + write), 25362432 B", "value": gbs, "unit": "GB/s",
            "ms_per_step": us / 1e3, "dtype": "u8", "config": {"workload": "hipMemcpyAsync D2D of 25362432 B"},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None}, "cpu_baseline": None}


def workload_cache(pkg, ctx, args):
    """Last-level cache residency under non-temporal reads (why the verify
    GEMMs load weights non-temporally): a 160 MB buffer D is read with plain
    loads until cache-resident, then 2 GB of other data T is read with plain
    or non-temporal loads, then D again.  D's re-read time against its
    resident and cold times shows whether T's reads allocated in the cache;
    T's time gives each policy's streaming rate.  Medians over --reps."""
    sink = ctx.alloc(16)
    DB, TB = 160 << 20, 2048 << 20
    d, t = ctx.alloc(DB), ctx.alloc(TB)

    def timed(buf, nbytes, variant):
        ctx.timer_mark(0)
        ctx.stream_read(buf, nbytes, variant, sink)
        ctx.timer_mark(1)
        ctx.sync()
        return ctx.timer_elapsed_ms(0, 1) * 1e3

    reps = max(3, min(args.reps, 20))
    for _ in range(2):
        timed(t, TB, 0)
        timed(d, DB, 0)
    rows = []
    for variant, label in ((0, "plain"), (4, "non-temporal")):
        hot, tt, after = [], [], []
        for _ in range(reps):
            timed(t, TB, 0)
            timed(d, DB, 0)
            hot.append(timed(d, DB, 0))
            tt.append(timed(t, TB, variant))
            after.append(timed(d, DB, 0))
        row = {"T_policy": label, "T_us": float(np.median(tt)), "T_GB/s": TB / float(np.median(tt)) / 1e3,
               "D_resident_us": float(np.median(hot)), "D_after_T_us": float(np.median(after))}
        log(f"T (2048 MB) read {label}: {row['T_us']:.1f} us ({row['T_GB/s']:.0f} GB/s); D (160 MB) resident "
            f"{row['D_resident_us']:.1f} us, D after T {row['D_after_T_us']:.1f} us")
        rows.append(row)
    cold = []
    for _ in range(reps):
        timed(t, TB, 0)
        cold.append(timed(d, DB, 0))
    log(f"D (160 MB) after a plain 2048 MB read of T: {float(np.median(cold)):.1f} us (cold)")
    for b in (d, t, sink):
        b.free()
    nt = rows[1]
    return {"metric": "2 GB streaming read rate with non-temporal loads (GB/s)", "value": nt["T_GB/s"], "unit": "GB/s",
            "ms_per_step": nt["T_us"] / 1e3, "dtype": "u8",
            "config": {"workload": "160 MB resident buffer, 2048 MB streamed past it with each load policy",
                       "table": rows, "D_cold_us": float(np.median(cold))},
            "roofline": {"bound": "hbm", "achieved": nt["T_GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": nt["T_GB/s"] / HBM_PEAK_GBS, "traffic": None}, "cpu_baseline": None}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--greedy", action="store_true")
    ap.add_argument("--batch", type=int, default=1, help="sequences stepped together (1 .. 8)")
    ap.add_argument("--temperature", type=float, default=0.8)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-steps", type=int, default=12, help="GPU steps recorded for the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="CPU work budget of the baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", choices=("step", "roofline", "gemm", "attention", "accept", "copy", "read", "q6k",
                                           "launch", "cache"),
                    default="step",
                    help="step: the speculative step (default); roofline: only the step's verify-GEMM roofline "
                         "measurement; gemm / attention / accept: one kernel alone; copy: counter calibration; "
                         "read: the streaming-read ceiling; q6k: the native Q6_K GEMM against fp16 at 32000x4096; "
                         "launch: the graph-replayed launch floor against grid-wide barriers; cache: last-level "
                         "cache residency under plain and non-temporal streaming reads")
    ap.add_argument("--reps", type=int, default=50, help="launches per timing (kernel workloads)")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch each step's kernels directly instead of replaying the captured graph")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the library measures the single-GPU "
              "speculative step; sharding across GPUs is not implemented.", file=sys.stderr)
        return 2
    pkg = load_package()
    synthetic_llama = importlib.import_module("universal_loader_amd.synthetic").synthetic_llama
    ctx = pkg.Context(0)
    if args.workload == "roofline":
        target, _ = synthetic_llama(pkg, ctx, dict(TARGET, max_ctx=CONTEXT + 64), pkg.Q4_K, seed=1)
        ids = weight_ids(pkg, ctx)
        M = K_SPEC + 1
        prompt = np.random.default_rng(args.seed).integers(0, TARGET["vocab"], 64).astype(np.int32)
        target.forward(prompt, 0)  # a K/V cache of 64 tokens, then
        target.forward(prompt[64 - M:], 64 - M, n_logits=1)  # the activations of a 6-row verify forward
        us, alg = instep_gemm_roofline(pkg, target, ids, M, 64 - M, reps=args.reps // 5 or 1)
        achieved = alg / (us * 1e-6) / 1e9
        log(f"in-step verify GEMMs (target, M={M}): {len(ids)} calls, {us:.2f} us/call, {alg / 1e6:.2f} MB/call, "
            f"{achieved:.0f} GB/s")
        us_x, _ = gemm_roofline(pkg, ctx, ids, M, reps=args.reps // 5 or 1)
        plain = alg / (us_x * 1e-6) / 1e9
        log(f"the same weights with plain fp16 X (ulspec_verify_gemm): {us_x:.2f} us/launch, {plain:.0f} GB/s")
        target.close()
        ctx.close()
        print(json.dumps({"metric": "verify-GEMM HBM GB/s, 7B-shape Q4_K target weights, M=6, in-step fused GEMMs",
                          "value": achieved, "unit": "GB/s",
                          "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                       "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic(), "avg_us": us,
                                       "algorithmic_bytes": alg,
                                       "plain_x": {"avg_us": us_x, "achieved": plain,
                                                   "frac": plain / HBM_PEAK_GBS}}}), flush=True)
        return 0
    if args.workload != "step":
        fn = {"gemm": workload_gemm, "attention": workload_attention, "accept": workload_accept,
              "copy": workload_copy, "read": workload_read, "q6k": workload_q6k,
              "launch": workload_launch, "cache": workload_cache}[args.workload]
        out = fn(pkg, ctx, args)
        base = {"n_gpus": 1, "steps": args.reps, "warmup": 1, "higher_is_better": True, "scaling": "weak",
                "vs_baseline": None, "data": "synthetic, seeded"}
        ctx.close()
        print(json.dumps(dict(base, **out)), flush=True)
        return 0
    use_cpu = not args.no_cpu
    cpu_steps = args.cpu_steps if use_cpu else 0
    cap = CONTEXT + (cpu_steps + args.warmup + args.steps) * (K_SPEC + 1) + 32
    B = args.batch
    if not 1 <= B <= 8:
        print(f"bench.py: --batch {B} (1 .. 8 sequences)", file=sys.stderr)
        return 2
    t0 = time.perf_counter()
    target, th = synthetic_llama(pkg, ctx, dict(TARGET, max_ctx=cap, n_seq=B), pkg.Q4_K, seed=1, keep_host=use_cpu)
    n_target_w = len(weight_ids(pkg, ctx))
    draft, dh = synthetic_llama(pkg, ctx, dict(DRAFT, max_ctx=cap, n_seq=B), pkg.Q4_K, seed=2, keep_host=use_cpu)
    t_synth = time.perf_counter() - t0
    log(f"weights synthesized and uploaded in {t_synth:.1f} s")
    rng = np.random.default_rng(args.seed)
    prompts = [rng.integers(0, TARGET["vocab"], CONTEXT).astype(np.int32) for _ in range(B)]
    s = pkg.sampling(greedy=True) if args.greedy else pkg.sampling(temperature=args.temperature)
    sp = pkg.Speculative(target, draft, K_SPEC, s, args.seed, n_seq=B)
    sp.set_graph(not args.no_graph)
    t0 = time.perf_counter()
    sp.prefill(prompts[0] if B == 1 else prompts)
    t_prefill = time.perf_counter() - t0
    log(f"prefill of {B} x {CONTEXT} tokens in {t_prefill:.1f} s")
    recorded, kv_t, kv_d = [], None, None
    if use_cpu:  # the CPU path on sequence 0
        kv_t = [target.kv_io(l, 0, 0, CONTEXT - 1) for l in range(TARGET["n_layers"])]
        kv_d = [draft.kv_io(l, 0, 0, CONTEXT - 1) for l in range(DRAFT["n_layers"])]
        for _ in range(cpu_steps):
            n = sp.seq_state(0)["n"]
            sp.steps(1)
            r = sp.last_step()
            if B > 1:
                r = {name: (a[0] if name != "n_accepted" else int(a[0])) for name, a in r.items()}
            recorded.append((n, r))
    sp.steps(args.warmup)
    st0 = sp.state()
    ctx.sync()
    ctx.timer_mark(0)
    t0 = time.perf_counter()
    sp.steps(args.steps)
    ctx.timer_mark(1)
    ctx.sync()
    wall = time.perf_counter() - t0
    ev_ms = ctx.timer_elapsed_ms(0, 1)
    st1 = sp.state()
    tokens = st1["n"] - st0["n"]
    accepted = st1["accepted"] - st0["accepted"]
    proposed = st1["proposed"] - st0["proposed"]
    log(f"{args.steps} steps: {tokens} tokens in {wall * 1e3:.1f} ms (events {ev_ms:.1f} ms), "
        f"accepted {accepted}/{proposed}")
    ids = [(i, info) for i, info in weight_ids(pkg, ctx)[:n_target_w]]
    Mv = (K_SPEC + 1) * B  # the target's verify rows per step
    seq = sp.tokens(seq=0) if use_cpu else None
    n_last = sp.seq_state(0)["n"]
    sp.close()
    plain = None
    if B == 1:
        # the step's own target GEMMs (fused prologues / epilogues, split X), on
        # the activations of the last verify forward, at its positions
        us, alg = instep_gemm_roofline(pkg, target, ids, Mv, n_last - Mv)
        us_x, _ = gemm_roofline(pkg, ctx, ids, Mv)
        plain = {"avg_us": us_x, "achieved": alg / (us_x * 1e-6) / 1e9,
                 "frac": alg / (us_x * 1e-6) / 1e9 / HBM_PEAK_GBS,
                 "kernel": "the same 129 weights through ulspec_verify_gemm with plain fp16 X"}
        log(f"plain-X verify GEMM (target, M={Mv}): {us_x:.2f} us/launch, {plain['achieved']:.0f} GB/s")
    else:
        us, alg = gemm_roofline(pkg, ctx, ids, Mv)
    achieved = alg / (us * 1e-6) / 1e9
    log(f"verify GEMM (target, M={Mv}): {len(ids)} weights, {us:.2f} us/call, {alg / 1e6:.2f} MB/call, "
        f"{achieved:.0f} GB/s")
    cpu = None
    if use_cpu:
        cpu = cpu_leg(pkg, args, th, dh, kv_t, kv_d, recorded, seq, cap, CONTEXT)
        log(f"cpu baseline: {cpu}")
    mode = "greedy" if args.greedy else f"temperature {args.temperature}, full vocabulary"
    out = {
        "metric": METRIC if B == 1 else METRIC.replace("bs=1", f"bs={B}"), "value": tokens / wall, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": wall * 1e3 / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_k weights x fp32 activations (split fp16 MFMA operands), fp32 accumulate",
        "data": "synthetic: random-init N(0, 0.02^2) weights quantized to Q4_K on the device, seeded prompt",
        "config": {"workload": f"speculative decoding step, 7B-shape Q4_K target (dim 4096, 32 layers, 32 heads, "
                               f"FFN 11008, vocab 32000) + draft (dim 2048, 16 layers, 16 heads, FFN 5632), k=5, "
                               f"bs={B}, context {CONTEXT}, {mode}",
                   "k": K_SPEC, "batch": B, "context": CONTEXT, "acceptance": accepted / max(1, proposed),
                   "tokens": tokens, "event_ms": ev_ms},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic() if B == 1 else None,
                     "kernel": ("the step's verify dequant-GEMMs as it runs them: the 129 target linears at M=6 "
                                "with fused prologues / epilogues and split fp16 X (gemm_ring_kernel for QKV, "
                                "gate/up, LM head; gemm_stream_kernel for O; gemm_slice_kernel + gemm_reduce_kernel "
                                "for down), us per GEMM call") if B == 1 else
                               f"verify dequant-GEMM (split-K gemm_slice_kernel + gemm_reduce_kernel), the 129 target "
                               f"weights, M={Mv}",
                     "avg_us": us, "algorithmic_bytes": alg, "plain_x": plain},
        "cpu_baseline": cpu,
    }
    target.close()
    draft.close()
    ctx.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
