"""Headline benchmark: Qwen3-0.6B-shaped bf16 decode at batch 1 on one MI355X.

A "step" is one greedy decode token (all 28 layers, the tied lm_head and argmax),
run by the persistent decode step (one cooperative launch for all K steps), with
weights, kept rows and the token already resident in HBM. The timed run is the C1 workload: a 128-token prompt (seed 1), then
K decode steps (K=32: context 128..160). Warmup runs W steps of an earlier
generation first. Prints one JSON line.

Also measured in the same run:
  * roofline of the dominant kernel: the persistent step itself (the decode call's
    only kernel), its algorithmic bytes (every weight once per token + the kept rows
    read) over its duration from HIP events on the runner's stream around the timed
    launch; traffic from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE passes;
  * the graph path's lm_head kernel (lanes, 151936 x 1024 bf16) against HBM
    (extra.graph_lm_head);
  * the whole step against HBM: 1,192,099,840 weight bytes + 114,688 B per kept
    position per token;
  * prefill GEMMs (M=2048, the C2 projection shapes) as a fraction of bf16 MFMA peak;
  * C3 paged attention (decode: 32 rows, ctx U[512, 8192]; prefill: 4 x 2048 causal),
    C4 fp8-e4m3 weight products (M 1, 8, 64) and C5 one MoE layer, each against its
    roofline (extra.c3_decode, c3_prefill, c4_fp8, c5_moe);
  * the CPU baseline: the oracle (a C restatement of tessera-interp) decoding a bounded
    sample of steps on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12          # B/s, MI355X
BF16_PEAK = 2.5e15         # FLOP/s dense, MI355X
WEIGHT_BYTES = 596_049_920 * 2
KV_BYTES_PER_POS = 28 * 2 * 8 * 128 * 2
PROMPT = 128


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=32)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--cpu-steps", type=int, default=8)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-gemm", action="store_true")
    p.add_argument("--no-rows", action="store_true", help="skip the C3/C4/C5 measurements")
    p.add_argument("--rows-only", action="store_true",
                   help="run only the C3/C4/C5 measurements (for kernel traces of those rows)")
    p.add_argument("--decode-only", action="store_true",
                   help="only the decode measurement (and a 256 MiB copy: the PMC yardstick)")
    p.add_argument("--gemm-only", action="store_true",
                   help="run only the C2 sweep at M=2048 (for kernel traces and PMC passes of tiled)")
    p.add_argument("--roofline-only", action="store_true",
                   help="run only the lm_head lanes kernel and a plain copy of known size "
                        "(the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes)")
    return p.parse_args()


def lm_head_roofline(torch, reps=20):
    """lanes on the lm_head shape, timed with HIP events on torch's current stream
    (the stream rules.lanes launches on)."""
    from tessera_amd import rules
    n, k = 151936, 1024
    g = torch.Generator(device="cuda").manual_seed(0)
    w = (torch.randn((n, k), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn((1, k), device="cuda", generator=g)
    gain = torch.ones(k, device="cuda")
    out = torch.empty((1, n), device="cuda")
    for _ in range(3):
        rules.lanes(x, w, gain=gain, out=out)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        rules.lanes(x, w, gain=gain, out=out)
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / reps
    nbytes = n * k * 2 + k * 4 * 2 + n * 4  # weights, x and gain, logits
    # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    # (profiles/lanes_lm_head_traffic.txt), scaled by a plain copy of known size.
    traffic = None
    prof = os.path.join(ROOT, "profiles", "lanes_lm_head_traffic.json")
    if os.path.exists(prof):
        traffic = json.load(open(prof))["traffic_bytes_per_launch"]
    return {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": nbytes / t / HBM_PEAK, "traffic": traffic,
            "kernel": "ts::gemv_kernel<1,8,f32 x,bf16 w> (lanes, lm_head 151936x1024, fused RmsNorm)",
            "bytes_per_launch": nbytes, "us_per_launch": t * 1e6}


def decode_roofline(m, steps, mean_ctx):
    """The persistent step over the timed decode call: one launch, `steps` tokens."""
    ms = m.decode_ms
    if ms <= 0:
        return None
    nbytes = int(steps * (WEIGHT_BYTES + KV_BYTES_PER_POS * mean_ctx))
    t = ms / 1e3
    traffic = None
    prof = os.path.join(ROOT, "profiles", "decode_step_traffic.json")
    if os.path.exists(prof):
        traffic = int(json.load(open(prof))["traffic_bytes_per_token"] * steps)
    return {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": nbytes / t / HBM_PEAK, "traffic": traffic,
            "kernel": "ts::decode_step_kernel (persistent greedy step: 28 layers, lm_head, pick; one launch)",
            "bytes_per_launch": nbytes, "us_per_launch": ms * 1e3, "steps_per_launch": steps}


def copy_reference(torch, nbytes=256 << 20, reps=5):
    """A plain device copy of known size: the yardstick that scales FETCH_SIZE and
    WRITE_SIZE counters to bytes."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return nbytes


def gemm_sweep(torch, reps=10):
    """C2 at M=2048: bf16 x and w, f32 accumulate, bf16 out; TFLOP/s per shape.
    Beside each shape, the vendor BLAS on the same operands and the same clock
    (torch.mm, hipBLASLt on this image): a reference for what the part reaches on the
    shape, not part of the measured path."""
    from tessera_amd import rules
    shapes = {"q": (1024, 2048), "kv": (1024, 1024), "o": (2048, 1024), "gate_up": (1024, 6144),
              "down": (3072, 1024), "lm_head": (1024, 151936)}
    M = 2048

    def clock(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / 1e3 / reps

    res, flops_all, t_all, tv_all = {}, 0.0, 0.0, 0.0
    for name, (K, N) in shapes.items():
        x = torch.randn((M, K), device="cuda").to(torch.bfloat16)
        w = torch.randn((N, K), device="cuda").to(torch.bfloat16)
        out = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
        t = clock(lambda: rules.tiled(x, w, out=out))
        tv = clock(lambda: torch.mm(x, w.t(), out=out))
        fl = 2.0 * M * N * K
        res[name] = {"us": round(t * 1e6, 2), "tflops": round(fl / t / 1e12, 1), "frac": round(fl / t / BF16_PEAK, 4),
                     "vendor_us": round(tv * 1e6, 2), "vendor_frac": round(fl / tv / BF16_PEAK, 4)}
        flops_all += fl
        t_all += t
        tv_all += tv
        del x, w, out
    return {"M": M, "shapes": res, "aggregate_frac": round(flops_all / t_all / BF16_PEAK, 4),
            "vendor_aggregate_frac": round(flops_all / tv_all / BF16_PEAK, 4), "vendor": "torch.mm (hipBLASLt)"}


def _graph_time(torch, fn, launches=20, replays=5):
    """Seconds per call of fn, from a HIP graph of `launches` calls replayed `replays`
    times (the per-node launch cost stays in; host launch overhead does not)."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            fn()
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / 1e3 / (launches * replays)


def c3_decode(torch):
    """C3 decode: 32 rows, ctx ~ U[512, 8192] (seed 2), 16 q / 8 kv heads x 128, bf16
    K/V in 16-row pages under a shuffled table; HBM-bound on the K/V bytes."""
    import numpy as np
    from tessera_amd import rules
    r = np.random.default_rng(2)
    rows, heads, kvh, width, page, keys = 32, 16, 8, 128, 16, 8192
    ctx = r.integers(512, 8193, rows)
    kept_pages = keys // page
    table = r.permutation(rows * kept_pages).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(2)
    k = torch.randn((rows * keys, kvh, width), device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn((rows * keys, kvh, width), device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn((rows, heads, width), device="cuda", generator=g)
    slots = torch.arange(rows, dtype=torch.int32, device="cuda")
    pos = torch.from_numpy((ctx - 1).astype(np.int32)).cuda()
    tab = torch.from_numpy(table).cuda()
    out = torch.empty_like(q)
    mp = int(ctx.max() - 1)
    fn = lambda: rules.attend_rows(q, k, v, slots, pos, keys=keys, scale=width ** -0.5, table=tab,
                                   kept_pages=kept_pages, page=page, max_position=mp, out=out)
    t = _graph_time(torch, fn, launches=10)
    nbytes = int(ctx.sum()) * kvh * width * 2 * 2 + rows * heads * width * 4 * 2 + rows * kept_pages * 4
    return {"bound": "hbm", "us": round(t * 1e6, 2), "bytes": nbytes, "GB_s": round(nbytes / t / 1e9, 1),
            "frac": round(nbytes / t / HBM_PEAK, 4), "sum_ctx": int(ctx.sum())}


def c3_prefill(torch):
    """C3 prefill: 4 sequences x 2048 causal, 16 q / 8 kv heads x 128, q and K/V bf16
    (K/V in shuffled 16-row pages), f32 out; MFMA-bound: 68.75 GFLOP (causal pairs
    incl. the diagonal)."""
    import numpy as np
    from tessera_amd import rules
    r = np.random.default_rng(4)
    seqs, n, heads, kvh, width, page = 4, 2048, 16, 8, 128, 16
    kept_pages = n // page
    table = r.permutation(seqs * kept_pages).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(4)
    k = torch.randn((seqs * n, kvh, width), device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn((seqs * n, kvh, width), device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn((seqs * n, heads, width), device="cuda", generator=g).to(torch.bfloat16)
    slots = torch.arange(seqs, dtype=torch.int32, device="cuda").repeat_interleave(n)
    pos = torch.arange(n, dtype=torch.int32, device="cuda").repeat(seqs)
    tab = torch.from_numpy(table).cuda()
    out = torch.empty(q.shape, device="cuda")
    fn = lambda: rules.flash_rows(q, k, v, slots, pos, keys=n, scale=width ** -0.5, table=tab,
                                  kept_pages=kept_pages, page=page, max_position=n - 1, out=out)
    t = _graph_time(torch, fn, launches=5)
    flops = seqs * heads * (n * (n + 1) // 2) * 4 * width
    res = {"bound": "mfma", "us": round(t * 1e6, 2), "tflops": round(flops / t / 1e12, 1),
           "frac": round(flops / t / BF16_PEAK, 4), "gflop": round(flops / 1e9, 2)}
    # Reference: torch's fused attention on the same sizes with dense (unpaged) K/V,
    # bf16 out (its flash backend on this image), not part of the measured path.
    del k, v, q, out
    try:
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel
        qd = torch.randn((seqs, heads, n, width), device="cuda", dtype=torch.bfloat16)
        kd = torch.randn((seqs, kvh, n, width), device="cuda", dtype=torch.bfloat16)
        vd = torch.randn((seqs, kvh, n, width), device="cuda", dtype=torch.bfloat16)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            run = lambda: F.scaled_dot_product_attention(qd, kd, vd, is_causal=True, enable_gqa=True)
            run()
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(10):
                run()
            e.record()
            torch.cuda.synchronize()
            tv = s.elapsed_time(e) / 1e3 / 10
        res.update({"vendor_us": round(tv * 1e6, 2), "vendor_frac": round(flops / tv / BF16_PEAK, 4),
                    "vendor": "torch scaled_dot_product_attention (flash backend, dense K/V)"})
    except Exception as e:  # the reference is optional: report why it is missing
        res["vendor"] = f"unavailable: {type(e).__name__}"
    return res


def c4(torch):
    """C4: e4m3 weights with a bf16 scale per output row (absmax/448 of N(0,0.02) rows),
    bf16 x; M in {1, 8, 64}; HBM-bound. Bytes N*K + 2N + 2MK + 2MN."""
    from tessera_amd import rules
    shapes = {"q_o": (4096, 4096), "k_v": (4096, 1024), "gate_up": (4096, 14336), "down": (14336, 4096)}
    g = torch.Generator(device="cuda").manual_seed(5)
    res, bytes_all, t_all = {}, 0.0, 0.0
    for name, (K, N) in shapes.items():
        w = torch.randn((N, K), device="cuda", generator=g) * 0.02
        scale = (w.abs().amax(1) / 448.0).to(torch.bfloat16)
        codes = (w / scale.float()[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
        del w
        for M in (1, 8, 64):
            x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
            out = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
            fn = lambda: rules.linear(x, codes, w_scale=scale, out=out)
            t = _graph_time(torch, fn, launches=20)
            nb = N * K + 2 * N + 2 * M * K + 2 * M * N
            res[f"{name}_M{M}"] = {"us": round(t * 1e6, 2), "frac": round(nb / t / HBM_PEAK, 4)}
            bytes_all += nb
            t_all += t
    return {"bound": "hbm", "shapes": res, "aggregate_frac": round(bytes_all / t_all / HBM_PEAK, 4)}


def blocks(torch):
    """Block-form weights on the m = 1 decode product (the seven forms of block.rs:251-291):
    the Qwen3 lm_head (151936 x 1024) and the Llama-3-8B-like gate (14336 x 4096) shapes,
    HBM-bound. Bytes = the packed tensor + 4K (x) + 4N (out)."""
    from tessera_amd import rules
    # form: (codes a block, bytes a block, scale bytes, head bytes, scale kind)
    forms = {"q8_0": (32, 34, 2, 0, "f16"), "mxfp8": (32, 33, 1, 0, "e8m0"), "int4_g32": (32, 18, 2, 0, "f16"),
             "q4_0": (32, 18, 2, 0, "f16"), "nvfp4": (16, 9, 1, 4, "e4m3"), "mxfp4": (32, 17, 1, 0, "e8m0"),
             "int4_g128": (128, 66, 2, 0, "f16")}
    res, bytes_all, t_all = {}, 0.0, 0.0
    for shape, (K, N) in {"lm_head": (1024, 151936), "gate": (4096, 14336)}.items():
        x = torch.randn((1, K), device="cuda")
        for form, (B, bb, sb, head, kind) in forms.items():
            rb = K // B * bb
            w = torch.randint(0, 256, (head + N * rb,), device="cuda", dtype=torch.uint8)
            blk = w[head:].view(N, K // B, bb)
            if kind == "f16":
                blk[:, :, 1] = 0x20                      # finite f16 scales
            elif kind == "e8m0":
                blk[:, :, 0] = 120
            else:
                blk[:, :, 0] &= 0x77                     # no e4m3 NaN scale
            if form == "mxfp8":
                blk[:, :, 1:] &= 0x77                    # no e4m3 NaN codes
            if head:
                w[:4] = torch.tensor([0, 0, 128, 63], dtype=torch.uint8, device="cuda")  # f32 1.0
            out = torch.empty((1, N), device="cuda")
            fn = lambda: rules.lanes(x, w, out=out, w_form=form, rows=N)
            t = _graph_time(torch, fn, launches=20)
            nb = head + N * rb + 4 * K + 4 * N
            res[f"{shape}_{form}"] = {"us": round(t * 1e6, 2), "frac": round(nb / t / HBM_PEAK, 4)}
            bytes_all += nb
            t_all += t
            del w
    return {"bound": "hbm", "shapes": res, "aggregate_frac": round(bytes_all / t_all / HBM_PEAK, 4)}


def c5(torch):
    """C5: one MoE layer, 4096 tokens, hidden 4096, 128 experts top-8 (softmax over the
    8 picked logits), FFN 1536, plus one shared expert; gate logits N(0,1) f32 (seed 3).
    Roofline max(557 us MFMA, 609 us HBM) = 0.609 ms."""
    from tessera_amd import rules
    tokens, hidden, experts, top, ffn = 4096, 4096, 128, 8, 1536
    g = torch.Generator(device="cuda").manual_seed(3)
    logits = torch.randn((tokens, experts), device="cuda", generator=g)
    h = torch.randn((tokens, hidden), device="cuda", generator=g).to(torch.bfloat16)
    w_in = torch.empty((experts, 2 * ffn, hidden), device="cuda", dtype=torch.bfloat16)
    w_out = torch.empty((experts, hidden, ffn), device="cuda", dtype=torch.bfloat16)
    for e in range(experts):  # N(0, 0.02) per expert, keeping the f32 temporaries small
        w_in[e] = (torch.randn((2 * ffn, hidden), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        w_out[e] = (torch.randn((hidden, ffn), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    s_in = (torch.randn((2 * ffn, hidden), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    s_out = (torch.randn((hidden, ffn), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    fn = lambda: rules.moe_layer(h, None, w_in, w_out, top=top, shared_in=s_in, shared_out=s_out, scores=logits)
    fn()
    torch.cuda.synchronize()
    reps = 3
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / reps
    flops = 2.0 * (tokens * top + tokens) * 3 * hidden * ffn
    wbytes = (experts + 1) * 3 * hidden * ffn * 2
    roof = max(flops / BF16_PEAK, wbytes / HBM_PEAK)
    del w_in, w_out
    return {"bound": "balanced", "ms": round(t * 1e3, 3), "tflops": round(flops / t / 1e12, 1),
            "weight_GB_s": round(wbytes / t / 1e9, 1), "roofline_ms": round(roof * 1e3, 3),
            "frac": round(roof / t, 4)}


def host_cpu():
    """The host the CPU baseline ran on: its logical cores, the ones this process may
    use, and the CPU model. The baseline uses at most 16 threads, the CPU share of one
    GPU on these boxes."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"host_cores": os.cpu_count(), "host_cores_usable": len(os.sched_getaffinity(0)), "cpu_model": model,
            "thread_cap": 16}


def cpu_baseline(model, prompt, steps, threads=None):
    """The oracle decoding `steps` tokens after the same prompt, kept rows copied from
    the device after its prefill; `threads` host cores (default: all, up to 16) via
    OpenMP over output columns, or 1 (the reference interpreter's single-threaded
    order, engine/ir/interp/src/round.rs:8-34)."""
    import numpy as np

    import oracle as O
    from oracle.qwen3 import Qwen3 as OracleQwen3, from_runner
    threads = threads or min(16, os.cpu_count() or 1)
    O.set_threads(threads)
    ref = OracleQwen3(from_runner(model))
    c = model.config
    for l in range(c.layers):
        k = O.bf16_widen(model.read("k_cache", l)).reshape(-1, c.kv_heads, c.head_dim)
        v = O.bf16_widen(model.read("v_cache", l)).reshape(-1, c.kv_heads, c.head_dim)
        pages = model.pages((PROMPT + c.page - 1) // c.page)
        for i in range(PROMPT):
            row = pages[i // c.page] * c.page + i % c.page
            ref.kv[l]["k"][i] = k[row]
            ref.kv[l]["v"][i] = v[row]
    tok = int(np.argmax(model.logits()))
    t0 = time.perf_counter()
    for i in range(steps):
        logits = ref.forward([tok], [PROMPT + i])
        tok = int(np.argmax(logits))
    dt = time.perf_counter() - t0
    how = f"OpenMP over output columns, {threads} threads" if threads > 1 else "one thread, reference order"
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port", **host_cpu(),
            "sample": f"{steps} greedy decode steps at context {PROMPT}..{PROMPT + steps} "
                      f"(oracle restatement of tessera-interp, {how})"}


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {a.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    if a.roofline_only:
        roof = lm_head_roofline(torch, reps=5)
        copy_reference(torch)
        print(json.dumps({"roofline": roof}), flush=True)
        return
    if a.gemm_only:
        print(json.dumps({"prefill_gemm": gemm_sweep(torch)}), flush=True)
        return
    if a.rows_only:
        print(json.dumps({"c3_decode": c3_decode(torch), "c3_prefill": c3_prefill(torch), "c4_fp8": c4(torch),
                          "c5_moe": c5(torch), "block_forms": blocks(torch)}), flush=True)
        return
    from tessera_amd.qwen3 import Qwen3, default_config
    cfg = default_config(max_context=PROMPT + max(a.steps, a.warmup) + 1, max_prompt=PROMPT)
    m = Qwen3(cfg, seed=0)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, PROMPT).astype(np.uint32)
    if a.warmup:
        m.prefill(prompt)
        m.decode(a.warmup)
    torch.cuda.synchronize()
    m.prefill(prompt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks = m.decode(a.steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    tok_s = a.steps / dt
    mean_ctx = PROMPT + (a.steps + 1) / 2
    step_bytes = WEIGHT_BYTES + KV_BYTES_PER_POS * mean_ctx
    roof = decode_roofline(m, a.steps, mean_ctx)
    if a.decode_only:
        copy_reference(torch)
        print(json.dumps({"value": round(tok_s, 2), "roofline": roof}), flush=True)
        m.close()
        return
    extra = {"graph_lm_head": lm_head_roofline(torch),
             "step_hbm_frac": round(step_bytes * tok_s / HBM_PEAK, 4),
             "step_bytes": int(step_bytes),
             "roofline_tok_s": round(HBM_PEAK / step_bytes, 1),
             "tokens_head": [int(t) for t in toks[:8]]}
    if not a.no_gemm:
        extra["prefill_gemm"] = gemm_sweep(torch)
    cpu = None
    if not a.no_cpu and a.cpu_steps > 0:
        cpu = cpu_baseline(m, prompt, a.cpu_steps)
        cpu["single_thread"] = cpu_baseline(m, prompt, 1, threads=1)
    m.close()
    if not a.no_rows:
        torch.cuda.empty_cache()
        extra["c3_decode"] = c3_decode(torch)
        extra["c3_prefill"] = c3_prefill(torch)
        extra["c4_fp8"] = c4(torch)
        extra["c5_moe"] = c5(torch)
        extra["block_forms"] = blocks(torch)
    line = {
        "metric": "decode tok/s + % HBM roofline (Qwen3-0.6B-shape b=1); prefill GEMM % MFMA peak",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(dt / a.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) bf16 weights, uniform random 128-token prompt (seed 1)",
        "config": {"workload": "C1 Qwen3-0.6B-shaped decode, batch 1, 128-token prompt then greedy steps",
                   "global_batch": 1, "seq_len": PROMPT + a.steps, "parallelism": "none (1 GPU)"},
        "roofline": roof, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
