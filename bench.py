"""Decode throughput of the gfx950 path on the Qwen2.5-0.5B-shaped synthetic
model (24 layers, hidden 896, 14/2 heads, FFN 4864, vocab 151936; Q4_K
projections, Q6_K attn_v/ffn_down, Q8_0 tied embedding), random-init
weights written as GGUF v3 from a fixed seed.

Workload per run: a 32-token prompt of uniform random ids is ingested
(engine.Forward per token, untimed), W greedy steps warm up, then K greedy
steps are timed.  A step is the reference's generate-loop body
(c2slm.go:153-222): vocab projection + repetition penalty 1.15 + argmax,
then Forward(best, pos); only the chosen id crosses to the host each step.

Prints one JSON line: value = K / wall time of the K steps on one GPU; the
roofline of the FFN launch, the decode launch that moves the most bytes
(k_ffn_block: RMSNorm + Q8_K + gate/up Q4_K GEMV + SwiGLU, then the Q6_K
down projection and the residual; eager launches back to back over the 24
layers' weights, paced by the GPU, between one pair of HIP events: the
per-dispatch time a kernel trace of `bench.py --only roofline` records);
and the CPU baseline (the reference's CPU path restated in C with its AVX2
kernels, on this host's cores, same workload; the scalar port beside it).
`extra` adds, outside the timed region: every decode kernel's time, bytes
and GB/s and the step's bytes and GB/s; the vocab kernel from HBM; the
operator microbench of the layer shapes (Q4_K/Q6_K x Q8_K GEMV and the Q8_K
quantiser, hot and with the weights rotated through 1 GiB of copies); the
batched prefill of a 512-token prompt; decode at long contexts (512 / 4096 /
32768 positions of N(0,1) K/V); decode and prefill with the real Q4_K_M
file's format mix (Q5_0 / Q8_0 / Q6_K); and decode of the Qwen3-1.7B shape
(head_dim 128, QK-norm).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PROMPT_LEN = 32
SEED = 20261201
PENALTY = 1.15  # c2slm.go:165,167 (the reference's constant)
# Algorithmic bytes of one vocab launch at 151936x896 Q8_0: weights 144,643,072
# + normX 3,584 + 64 window ids 256 + the chosen id 4.
VOCAB_BYTES = 144_643_072 + 3_584 + 256 + 4


def synth_model(path: str):
    from c2slm_amd import gguf as G
    if not os.path.exists(path):
        G.write_synthetic_model(path, G.QWEN05B, seed=SEED)
    return path


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """The reference's pool size nw = min(GOMAXPROCS, 32) (engine/pool.go:47-53)
    over the cores this process may use: its affinity set, or the thread
    count the host grants it (OMP_NUM_THREADS) when that is smaller."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, min(32, n))


def cpu_baseline(gf, prompt, steps, im_end, eos, runs: int = 5, single_steps: int = 16):
    """The reference's CPU path on this host, as its C restatement with the
    reference's AVX2 kernels (oracle/c2slm_avx2.c: VPMADDUBSW / VPMADDWD
    Q4_K and Q6_K dots, the 8-lane float Q8_0 dot; the rest of the oracle's
    C), the reference's pool size (nw = min(32, cores granted) workers, rows
    split per worker, inline below 256 rows): after an untimed prompt ingest,
    `steps` greedy steps timed, the median of `runs` runs; beside it the
    scalar port (the oracle's scalar integer dots) on the same pool, and the
    AVX2 path on one thread for `single_steps` steps."""
    from oracle import oracle as O
    threads = cpu_threads()

    def rate(nt, n, avx2):
        orc = O.OracleEngine(gf, max_ctx=512, n_threads=nt, avx2_dots=avx2)
        orc.ingest_from(0, prompt)
        t0 = time.perf_counter()
        toks = orc.generate(n, -1, -1, PENALTY)  # run exactly n steps
        dt = time.perf_counter() - t0
        orc.close()
        return len(toks) / dt, dt

    rs = [rate(threads, steps, True) for _ in range(runs)]
    med = float(np.median([r for r, _ in rs]))
    scalar, scalar_dt = rate(threads, steps, False)
    one, one_dt = rate(1, single_steps, True)
    return {"value": round(med, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "implementation": "C restatement of the reference's AVX2 path (oracle/c2slm_avx2.c + oracle/c2slm_oracle.c)",
            "sample": f"{PROMPT_LEN}-token prompt ingest untimed, then {steps} greedy steps timed, median of {runs} "
                      f"runs ({sum(d for _, d in rs):.1f} s), {threads} OpenMP threads = min(32, cores granted)",
            "scalar_port_tok_s": round(scalar, 3),
            "scalar_port_sample": f"the same workload with the oracle's scalar integer dots, one run ({scalar_dt:.1f} s)",
            "single_thread_tok_s": round(one, 3), "single_thread_sample": f"{single_steps} steps ({one_dt:.1f} s)",
            "nproc": os.cpu_count(), "cpu_model": cpu_model(), "runs_tok_s": [round(r, 3) for r, _ in rs]}


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` as measured by the rocprofv3 --pmc
    passes (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration)
    recorded in profiles/roofline_*.md (the roofline command's own passes)
    or profiles/*_traffic.txt; None when no record names it."""
    import glob
    paths = sorted(glob.glob(os.path.join(ROOT, "profiles", "roofline_*.md")))
    paths += sorted(glob.glob(os.path.join(ROOT, "profiles", "*_traffic.txt")))
    for path in paths:
        try:
            with open(path, encoding="utf-8") as f:
                for line in f:
                    if not line.startswith("traffic_bytes_per_launch") or "=" not in line:
                        continue
                    head, val = line.split("=", 1)
                    name = head.strip()[len("traffic_bytes_per_launch"):].strip()
                    if name == f"[{kernel}]" or (not name and kernel == "vocab"):
                        return int(val.strip())
        except OSError:
            pass
    return None


def kernel_bytes(gf, desc, T: float) -> dict:
    """Algorithmic bytes per launch of each decode kernel at T attended
    positions (the reference's floor semantics: a K-quant row of 896 columns
    is 3 super-blocks): weights + inputs + outputs + parameters."""
    from c2slm_amd import gguf as G
    tm = gf.tensor_map
    E, F, KVd = desc.n_embd, desc.n_ff, desc.n_kv_heads * desc.head_dim

    def w(name):
        ti = tm[name]
        return G.row_bytes(ti.ggml_type, int(ti.dims[0])) * int(ti.dims[1])

    def avg(fn):
        return sum(fn(i) for i in range(desc.n_layers)) / desc.n_layers

    q = avg(lambda i: w(f"blk.{i}.attn_q.weight") + w(f"blk.{i}.attn_k.weight") + w(f"blk.{i}.attn_v.weight"))
    o = avg(lambda i: w(f"blk.{i}.attn_output.weight"))
    gu = avg(lambda i: w(f"blk.{i}.ffn_gate.weight") + w(f"blk.{i}.ffn_up.weight"))
    dn = avg(lambda i: w(f"blk.{i}.ffn_down.weight"))
    out = tm.get("output.weight", tm["token_embd.weight"])
    vocab_w = G.row_bytes(out.ggml_type, int(out.dims[0])) * int(out.dims[1])
    b = {
        "qkv": int(q + 4 * (E + E + 2 * (E + 2 * KVd))),          # + x, norm w, bias, q|k|v out
        "attn": int(4 * 2 * KVd * T + 4 * (2 * (E + 2 * KVd) + E)),  # K,V rows + q|k|v in, K/V store, out
        "attn_out": int(o + 4 * (E + 2 * E)),                      # + attn in, X read and written
        "ffn_in": int(gu + 4 * (E + E + F)),                       # + x, norm w, h out
        "ffn_out": int(dn + 4 * (F + 2 * E)),                      # + h in, X read and written
        "final_norm": int(4 * 3 * E),
        "vocab": int(vocab_w + 4 * E + 4 * 64 + 4),                # + normX, window ids, chosen id
    }
    # the fused launches: the sum of their parts (the handed-over q|k|v,
    # attention output and h counted once written, once read, as between
    # kernels; the FFN's residual add, which the next k_attn_block does from
    # the down projection's 19 terms per row, counted with the FFN)
    b["attn_block"] = b["qkv"] + b["attn"] + b["attn_out"]
    b["attn_oproj"] = b["attn"] + b["attn_out"]
    b["ffn_block"] = b["ffn_in"] + b["ffn_out"]
    return b


def step_launches(n_layers: int) -> dict:
    """Launches of each decode kernel per step.  The Qwen2.5-0.5B shape has
    the fused attention launches (k_attn_block on layers past 0, qkv then
    k_attn_oproj on layer 0) and the FFN as one launch (k_ffn_block) whose
    residual add the next k_attn_block, or after the last layer the final
    norm, does, unless C2H_NO_FUSE selects the separate forms (=1: every
    kernel on its own; =qkv: qkv on its own, attention and the o-projection
    fused, the FFN's two launches apart but on the last layer; =ffn: the
    FFN's two launches apart)."""
    nf = os.environ.get("C2H_NO_FUSE", "")
    L = n_layers
    n = dict(qkv=1, attn=0, attn_out=0, attn_block=L - 1, attn_oproj=1, ffn_in=0, ffn_out=0, ffn_block=L,
             final_norm=1, vocab=1)
    if nf in ("1", "ffn"):
        n.update(ffn_in=L, ffn_out=L, ffn_block=0)
    if nf == "1":
        n.update(qkv=L, attn=L, attn_out=L, attn_block=0, attn_oproj=0)
    elif nf == "qkv":
        n.update(qkv=L, attn_oproj=L, attn_block=0, ffn_in=L - 1, ffn_out=L - 1, ffn_block=1)
    return n


# The roofline line's kernel: the decode launch with the most bytes (the
# layer's FFN: two 4864 x 896 Q4_K matrices and a 896 x 4864 Q6_K one),
# fixed so the line does not depend on which kernel a run's timings make the
# largest; ffn_in (the two Q4_K matrices) where C2H_NO_FUSE runs the FFN's
# launches apart.
ROOFLINE_KERNEL = "ffn_in" if os.environ.get("C2H_NO_FUSE", "") in ("1", "ffn") else "ffn_block"

KERNEL_NAMES = {"qkv": "k_gemv_row<3, PRO_NORM, MODE_BIAS>", "attn": "k_attn_core",
                "attn_out": "k_gemv_row<3, PRO_QUANT, MODE_RESID>", "ffn_in": "k_gemv_row<3, PRO_NORM, MODE_SWIGLU>",
                "ffn_out": "k_gemv_row<19, PRO_QUANT, MODE_RESID>", "final_norm": "k_rmsnorm",
                "vocab": "k_vocab<28>", "attn_block": "k_attn_block<TIER, 3>", "attn_oproj": "k_attn_oproj<TIER, 3>",
                "ffn_block": "k_ffn_block<3, 19>"}


def decode_kernels(ctx, gf, desc, vocab_ms, step_ms, T, iters: int = 96):
    """Each decode kernel's device time per launch (c2h_time_layer_kernel,
    `iters` launches over the layers' weights, one pair of HIP events):
    `us` eager launches back to back, paced by the GPU (the host enqueues
    them all behind a short wait on the device; a rocprofv3 kernel trace of
    the same launches records per-dispatch durations within a few per cent
    of it), `us_graph` the same launches captured in one graph (the figure a
    step's replay sees); its algorithmic bytes and GB/s at `us`, and its
    share of the step at `us_graph`.  The separate attention kernels are
    timed too where the step runs them fused (launches_per_step 0)."""
    from c2slm_amd import _lib as H
    nbytes = kernel_bytes(gf, desc, T)
    per_step = step_launches(desc.n_layers)
    out = {}
    for k in ctx.KERNELS:
        try:
            us = ctx.time_layer_kernel(k, iters) * 1e3
            usg = ctx.time_layer_kernel(k, iters, captured=True) * 1e3
        except H.C2hError:  # a fused launch this model or C2H_NO_FUSE does not run
            continue
        out[k] = {"us": round(us, 3), "us_graph": round(usg, 3)}
    out["vocab"] = {"us": round(vocab_ms * 1e3, 3), "us_graph": round(vocab_ms * 1e3, 3)}
    for k, v in out.items():
        gbs = nbytes[k] / (v["us"] * 1e-6) / 1e9
        v.update(bytes=nbytes[k], gb_s=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4),
                 launches_per_step=per_step[k],
                 share_of_step=round(v["us_graph"] * per_step[k] / (step_ms * 1e3), 4), kernel=KERNEL_NAMES[k])
    return out


def roofline_timing(ctx, gf, desc, prompt, iters: int):
    """The roofline line's kernel (ffn_block) on a fixed state: the prompt
    ingested by one batched prefill (which launches no decode layer kernel), then
    `iters` eager launches back to back over the 24 layers' weights, paced by
    the GPU, between one pair of HIP events.  The kernel's time depends on
    its input (the exact RMSNorm sum takes more rounds on some rows), so the
    bench line and `bench.py --only roofline` (the profiled command) time it
    on the same state."""
    ctx.prefill(prompt, 0, want_normx=False)
    us = ctx.time_layer_kernel(ROOFLINE_KERNEL, iters) * 1e3
    nb = kernel_bytes(gf, desc, PROMPT_LEN + 1)[ROOFLINE_KERNEL]
    return us, nb


def producer_consumer_wait(ctx, n_launch: int = 100, reps: int = 5):
    """The cost of a producer -> consumer dependency inside one launch
    against a kernel boundary (c2h_time_producer_consumer): for the
    producer/consumer workgroup counts of the decode layer's boundaries
    (qkv 129 -> attention, attention 14 -> attn_out, ffn_out 150 -> the
    next qkv, ffn_in 232 -> ffn_out), without and with 400 dependent float
    steps of producer work, under both wait protocols (per-XCD counters;
    outputs tagged with the launch number), µs per fused launch and per
    split launch pair; plus the launch floor at those grids."""
    out = {"launch_floor_us": {g: round(ctx.launch_floor(240, g, 5), 3) for g in (57, 185, 279, 382)}}
    for proto, name in ((0, "counters"), (1, "tagged")):
        for work in (0, 400):
            for p, c in ((14, 43), (129, 56), (150, 129), (232, 150)):
                f, sp = ctx.time_producer_consumer(p, c, work, n_launch, reps, proto)
                out[f"{name}_P{p}_C{c}_work{work}"] = {"fused_us": round(f, 3), "split_pair_us": round(sp, 3),
                                                       "saving_us": round(sp - f, 3)}
    return out


def layer_microbench(ctx, iters: int = 200, rotate_mib: int = 1024):
    """The operator GEMVs at every layer shape (tensor/ops_test.go:143-171's
    benchmark shapes; BASELINE distributions) and the Q8_K quantiser, hot
    (one copy, from the caches) and cold (rotating over 1 GiB of copies, from
    HBM).  Bytes as the reference reads them: W + Q8_K row + y; the
    quantiser reads x and writes its Q8_K blocks."""
    from c2slm_amd import _lib as H
    from c2slm_amd import gguf as G
    rng = np.random.default_rng(SEED + 5)
    out = {}
    shapes = [("q4k_896x896", H.Q4_K, 896, 896), ("q4k_128x896", H.Q4_K, 128, 896),
              ("q4k_4864x896", H.Q4_K, 4864, 896), ("q4k_896x4864", H.Q4_K, 896, 4864),
              ("q6k_896x4864", H.Q6_K, 896, 4864)]
    for name, t, rows, cols in shapes:
        nb = cols // 256
        w = (G.synth_q4_k if t == H.Q4_K else G.synth_q6_k)(rng, rows * nb)
        xq = ctx.quantize_q8k(rng.standard_normal(cols).astype(np.float32))
        nbytes = rows * nb * (144 if t == H.Q4_K else 210) + nb * 292 + rows * 4
        rec = {"rows": rows, "cols": cols, "bytes": nbytes}
        for mode, rot in (("hot", 0), ("cold", rotate_mib << 20)):
            ms = ctx.time_gemv(t, w, xq, rows, cols, iters, rot)
            gbs = nbytes / (ms * 1e-3) / 1e9
            rec[mode] = {"us": round(ms * 1e3, 3), "gb_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        out[name] = rec
    for cols in (896, 4864):
        x = rng.standard_normal(cols).astype(np.float32)
        nb = cols // 256
        nbytes = nb * 256 * 4 + nb * 292
        rec = {"cols": cols, "bytes": nbytes}
        for mode, rot in (("hot", 0), ("cold", rotate_mib << 20)):
            ms = ctx.time_quantize_q8k(x, iters, rot)
            rec[mode] = {"us": round(ms * 1e3, 3), "gb_s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        out[f"quantize_q8k_{cols}"] = rec
    return out


def copy_calibration(ctx, mib: int, reps: int = 5):
    """A plain device-to-device copy of `mib` MiB (k_copy16), `reps` times:
    under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE per dispatch against
    the known size gives the counters' scale factor."""
    ms = ctx.copy_bench(mib << 20, reps)
    print(f"copy calibration: {reps} x {mib} MiB device copies, {ms:.4f} ms each "
          f"({2 * (mib << 20) / (ms * 1e-3) / 1e9:.1f} GB/s read+write)", file=sys.stderr)


def prefill_rate(ctx, desc, reps: int = 5):
    """Batched prefill of a 512-token prompt of uniform random ids at position
    0 (c2h_prefill: int8 MFMA GEMMs, causal attention, KV population), timed
    on the host around the synchronous call; effective int8 rate of its
    projections (floor(cols/256)*256 columns per row, as the reference's
    K-quant rows are read)."""
    m = 512
    toks = np.random.default_rng(SEED + 1).integers(0, desc.n_vocab, m).astype(np.int32)
    ctx.prefill(toks, 0, want_normx=False)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        ctx.prefill(toks, 0, want_normx=False)
        ts.append(time.perf_counter() - t0)
    E, F = desc.n_embd, desc.n_ff
    KV = desc.n_kv_heads * desc.head_dim
    ce, cf = E // 256 * 256, F // 256 * 256
    macs = desc.n_layers * (E * ce + 2 * KV * ce + E * ce + 2 * F * ce + E * cf) * m
    best = min(ts)
    return {"tokens": m, "ms": round(best * 1e3, 3), "tok_s": round(m / best, 1),
            "int8_macs": macs, "effective_int8_tops": round(2 * macs / best / 1e12, 2),
            "ms_all": [round(t * 1e3, 3) for t in ts]}


def float_x_dots(ctx, iters: int = 20, flush_mib: int = 512):
    """The float-x row dots (c2h_gemv_f32: DispatchGEMV without a pool;
    c2h_logits_ids: ComputeLogits with a target list) over a 151936 x 896
    matrix of each format (random blocks; K-quant rows floor to 768
    columns), the matrix evicted from the last-level cache by a 512 MiB copy
    before each launch; plus a 64-id restricted-logits launch on the Q8_0
    matrix.  GB/s counts the matrix bytes the dots read."""
    from c2slm_amd import _lib as H
    from c2slm_amd import gguf as G
    rng = np.random.default_rng(SEED + 3)
    V, E = 151936, 896
    x = rng.normal(size=E).astype(np.float32)
    out = {}
    q8 = None
    for name, typ, synth, qk, bs in (("q8_0", H.Q8_0, G.synth_q8_0, 32, 34), ("q6_k", H.Q6_K, G.synth_q6_k, 256, 210),
                                     ("q4_k", H.Q4_K, G.synth_q4_k, 256, 144), ("q5_0", H.Q5_0, G.synth_q5_0, 32, 22)):
        nb = E // qk
        w = synth(rng, V * nb)
        ms, _ = ctx.time_dot_rows(typ, w, x, V, E, iters=iters, flush_bytes=flush_mib << 20)
        nbytes = V * nb * bs
        out[name] = {"ms": round(ms, 4), "matrix_bytes": nbytes, "gb_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if typ == H.Q8_0:
            q8 = w
    ids = rng.integers(0, V, 64).astype(np.int32)
    ms, _ = ctx.time_dot_rows(H.Q8_0, q8, x, V, E, ids=ids, iters=iters, flush_bytes=flush_mib << 20)
    out["logits_64_ids_q8_0_us"] = round(ms * 1e3, 2)
    return out


def long_context(gf, im_end, eos, lengths, steps: int = 16):
    """Decode at long contexts (the KV cache pre-filled with N(0,1) keys and
    values, token ids uniform): device-fed greedy steps whose last one
    attends `n` positions, per n."""
    from c2slm_amd import _lib as H
    top = max(lengths)
    desc = H.desc_from_gguf(gf, max_ctx=max(top, 1024))
    ctx = H.Ctx(desc)
    H.load_gguf_into(ctx, gf)
    rng = np.random.default_rng(SEED + 2)
    for which in (0, 1):
        for layer in range(desc.n_layers):
            for h in range(desc.n_kv_heads):
                ctx.set_kv(which, layer, h, 0, rng.standard_normal((top, desc.head_dim), dtype=np.float32))
    ctx.set_token_ids(0, rng.integers(0, desc.n_vocab, top).astype(np.int32))
    out = {}
    for n in lengths:
        pos = n - steps
        ctx.forward(11, pos - 1, want_normx=False)
        ms = ctx.time_steps(pos, steps, PENALTY, im_end, eos)
        out[str(n)] = {"ms_per_step": round(ms, 4), "tok_s": round(1000.0 / ms, 1)}
    ctx.close()
    return out


def real_formats(tmpdir, im_end, eos, steps: int = 64):
    """The published Qwen2.5-0.5B-Instruct Q4_K_M file's format mix (Q5_0
    q/k/o/gate/up, Q8_0 attn_v, Q6_K ffn_down) at the same shape, random-init:
    device-fed greedy steps after a 32-token batched prefill, and the
    512-token prefill."""
    from c2slm_amd import _lib as H
    from c2slm_amd import gguf as G
    path = os.path.join(tmpdir, "qwen05b_real_formats.gguf")
    G.write_synthetic_model(path, G.QWEN05B_REAL_FORMATS, seed=SEED + 3)
    gf = G.GGUFFile(path)
    desc = H.desc_from_gguf(gf, max_ctx=1024)
    ctx = H.Ctx(desc)
    H.load_gguf_into(ctx, gf)
    prompt = np.random.default_rng(SEED).integers(0, desc.n_vocab, PROMPT_LEN).astype(np.int32)
    ctx.prefill(prompt, 0, want_normx=False)
    ms = ctx.time_steps(PROMPT_LEN, steps, PENALTY, im_end, eos)
    pf = prefill_rate(ctx, desc, 3)
    ctx.close()
    del gf
    os.remove(path)
    return {"formats": "Q5_0 q/k/o/gate/up, Q8_0 attn_v, Q6_K ffn_down, Q8_0 embedding",
            "decode_ms_per_step": round(ms, 4), "decode_tok_s": round(1000.0 / ms, 1),
            "prefill_512_ms": pf["ms"], "prefill_512_tok_s": pf["tok_s"]}


def qwen3_decode(tmpdir, im_end, eos, steps: int = 64, device_fed_only: bool = False):
    """The Qwen3-1.7B shape (28 layers, hidden 2048, 16/8 heads of 128, FFN
    6144, per-head QK-norm, tied Q8_0 embedding; Q4_K / Q6_K projections),
    random-init: a 32-token prompt (one forward per token at head_dim 128),
    then greedy steps timed on the host around synchronous c2h_step calls,
    as the main line, and device-fed (c2h_time_steps); algorithmic bytes of
    a step at the mean attended position.  device_fed_only: the warm-up and
    timed steps fed on the device only (graph replays without c2h_step, the
    form a rocprofv3 kernel trace runs through)."""
    from c2slm_amd import _lib as H
    from c2slm_amd import gguf as G
    path = os.path.join(tmpdir, "qwen3_1_7b_synth.gguf")
    G.write_synthetic_model(path, G.QWEN3_1_7B, seed=SEED + 7)
    gf = G.GGUFFile(path)
    desc = H.desc_from_gguf(gf, max_ctx=1024)
    ctx = H.Ctx(desc)
    H.load_gguf_into(ctx, gf)
    prompt = np.random.default_rng(SEED).integers(0, desc.n_vocab, PROMPT_LEN).astype(np.int32)
    ctx.set_token_ids(0, prompt)
    ctx.prefill(prompt, 0, want_normx=False)
    pos = PROMPT_LEN
    if device_fed_only:
        fed_ms = ctx.time_steps(pos, 8 + steps, PENALTY, im_end, eos)
        ctx.close()
        del gf
        os.remove(path)
        return {"shape": "Qwen3-1.7B", "positions": [pos, pos + 8 + steps - 1],
                "device_fed_ms_per_step": round(fed_ms, 4), "device_fed_tok_s": round(1000.0 / fed_ms, 1)}
    for _ in range(8):
        ctx.step(pos, PENALTY, im_end, eos)
        pos += 1
    ctx.normx()
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.step(pos, PENALTY, im_end, eos)
        pos += 1
    ctx.sync()  # the last step's forward completes inside the timed region
    ms = (time.perf_counter() - t0) * 1e3 / steps
    fed_ms = ctx.time_steps(pos, steps, PENALTY, im_end, eos)
    kb = kernel_bytes(gf, desc, pos - steps / 2)
    step_bytes = (desc.n_layers * sum(kb[k] for k in ("qkv", "attn", "attn_out", "ffn_in", "ffn_out"))
                  + kb["final_norm"] + kb["vocab"])
    ctx.close()
    del gf
    os.remove(path)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    return {"shape": "Qwen3-1.7B: 28 layers, hidden 2048, 16/8 heads x 128, FFN 6144, QK-norm, vocab 151936",
            "ms_per_step": round(ms, 4), "tok_s": round(1000.0 / ms, 1),
            "device_fed_ms_per_step": round(fed_ms, 4), "device_fed_tok_s": round(1000.0 / fed_ms, 1),
            "step_bytes": int(step_bytes), "gb_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--model", default=None, help="GGUF path (default: synthesise the seeded model)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--max-ctx", type=int, default=16384)
    ap.add_argument("--vocab-iters", type=int, default=50, help="launches in each vocab timing")
    ap.add_argument("--pipelined-iters", type=int, default=64, help="steps in the pipelined (no host sync) timing")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run plain device copies of this size (counter calibration under rocprofv3 --pmc)")
    ap.add_argument("--long-context", default="512,4096,32768",
                    help="context lengths of the long-context decode lines ('' to skip)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 512-token prefill line")
    ap.add_argument("--no-real-formats", action="store_true", help="skip the real-model format line")
    ap.add_argument("--no-float-dots", action="store_true", help="skip the float-x row-dot timings")
    ap.add_argument("--no-microbench", action="store_true", help="skip the layer-shape operator microbench")
    ap.add_argument("--no-qwen3", action="store_true", help="skip the Qwen3-1.7B-shape decode line")
    ap.add_argument("--kernel-iters", type=int, default=96, help="launches in each decode-kernel timing")
    ap.add_argument("--kernel-pos", type=int, default=None,
                    help="with --only kernels: greedy steps after the prompt up to this position, so attention "
                         "covers pos+1 positions (default: the decode line's last position, prompt + warmup + steps)")
    ap.add_argument("--only", choices=["prefill", "long", "float-dots", "real-formats", "vocab", "microbench",
                                       "kernels", "qwen3", "qwen3-steps", "roofline", "wait", "steps"],
                    default=None,
                    help="run just the prefill reps or just the long-context decode (profiler runs); "
                         "prints their JSON object, not the bench line")
    ap.add_argument("--prefill-reps", type=int, default=5)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    from c2slm_amd import _lib as H
    from c2slm_amd import gguf as G

    tmpdir = None
    path = args.model
    if path is None:
        tmpdir = tempfile.mkdtemp(prefix="c2slm_bench_")
        path = os.path.join(tmpdir, "qwen05b_synth.gguf")

    def cleanup():
        if tmpdir:
            try:
                os.remove(path)
                os.rmdir(tmpdir)
            except OSError:
                pass

    synth_model(path)
    gf = G.GGUFFile(path)
    _, im_end, eos = G.special_token_ids(gf)
    if args.only == "real-formats":
        rdir = tempfile.mkdtemp(prefix="c2slm_bench_")
        print(json.dumps({"real_formats": real_formats(rdir, im_end, eos)}))
        os.rmdir(rdir)
        cleanup()
        return
    if args.only in ("qwen3", "qwen3-steps"):
        rdir = tempfile.mkdtemp(prefix="c2slm_bench_")
        print(json.dumps({"qwen3_1_7b_decode": qwen3_decode(rdir, im_end, eos,
                                                            device_fed_only=args.only == "qwen3-steps")}))
        os.rmdir(rdir)
        cleanup()
        return
    if args.only in ("float-dots", "microbench", "wait"):
        ctx = H.Ctx(None)
        if args.only == "float-dots":
            print(json.dumps({"float_x_dots": float_x_dots(ctx)}))
        elif args.only == "wait":
            print(json.dumps({"producer_consumer_wait": producer_consumer_wait(ctx)}))
        else:
            print(json.dumps({"layer_microbench": layer_microbench(ctx)}))
        ctx.close()
        cleanup()
        return
    if args.only == "long":
        lengths = [int(x) for x in args.long_context.split(",") if x]
        print(json.dumps({"long_context_decode": long_context(gf, im_end, eos, lengths)}))
        cleanup()
        return
    desc = H.desc_from_gguf(gf, max_ctx=args.max_ctx)
    ctx = H.Ctx(desc)
    H.load_gguf_into(ctx, gf)
    if args.only == "prefill":
        print(json.dumps({"prefill_512": prefill_rate(ctx, desc, args.prefill_reps)}))
        ctx.close()
        cleanup()
        return
    rng = np.random.default_rng(SEED)
    prompt = rng.integers(0, desc.n_vocab, PROMPT_LEN).astype(np.int32)
    if args.only == "kernels":  # the decode kernels alone (profiler runs)
        ctx.set_token_ids(0, prompt)
        for p, t in enumerate(prompt):
            ctx.forward(int(t), p, want_normx=False)
        kpos = PROMPT_LEN + args.warmup + args.steps if args.kernel_pos is None else args.kernel_pos
        for p in range(PROMPT_LEN, kpos):
            ctx.step(p, PENALTY, im_end, eos)
        ctx.sync()
        out = {}
        for k in ctx.KERNELS:
            try:
                out[k] = [round(ctx.time_layer_kernel(k, args.kernel_iters, captured=g) * 1e3, 3)
                          for g in (False, True)]
            except H.C2hError:  # a fused launch this run does not have
                pass
        out["attended_positions"] = ctx.seq_len + 1
        if args.copy_calib_mib:
            copy_calibration(ctx, args.copy_calib_mib)
        print(json.dumps({"decode_kernels_us_eager_graph": out}))
        ctx.close()
        cleanup()
        return
    if args.only == "roofline":  # the roofline line's timing alone (profiler runs)
        us, nb = roofline_timing(ctx, gf, desc, prompt, args.kernel_iters)
        if args.copy_calib_mib:
            copy_calibration(ctx, args.copy_calib_mib)
        print(json.dumps({"roofline_kernel": f"{ROOFLINE_KERNEL}: {KERNEL_NAMES[ROOFLINE_KERNEL]}",
                          "launches_timed": args.kernel_iters, "us_per_launch": round(us, 3), "bytes_per_launch": nb,
                          "achieved_gbs": round(nb / (us * 1e-6) / 1e9, 1),
                          "frac": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}))
        ctx.close()
        cleanup()
        return
    if args.only == "steps":  # the decode workload's steps fed on the device: graph replays only (profiler runs)
        ctx.set_token_ids(0, prompt)
        for p, t in enumerate(prompt):
            ctx.forward(int(t), p, want_normx=False)
        n = args.warmup + args.steps
        ms = ctx.time_steps(PROMPT_LEN, n, PENALTY, im_end, eos)
        print(json.dumps({"device_fed_steps": {"positions": [PROMPT_LEN, PROMPT_LEN + n - 1],
                                               "ms_per_step": round(ms, 4), "tok_s": round(1000.0 / ms, 1)}}))
        ctx.close()
        cleanup()
        return
    if args.only == "vocab":  # the vocab kernel alone (profiler runs)
        ctx.set_token_ids(0, prompt)
        for p, t in enumerate(prompt):
            ctx.forward(int(t), p, want_normx=False)
        ms = ctx.time_vocab(args.vocab_iters, PROMPT_LEN, in_step=2)
        if args.copy_calib_mib:
            copy_calibration(ctx, args.copy_calib_mib)
        print(json.dumps({"vocab_ms_alternating": round(ms, 5),
                          "achieved_gbs": round(VOCAB_BYTES / (ms * 1e-3) / 1e9, 1)}))
        ctx.close()
        cleanup()
        return

    # first on the fresh context: the roofline kernel on the state bench.py
    # --only roofline reproduces (model uploaded, the prompt ingested by a
    # batched prefill); its time depends on the caches' contents, which the
    # later work changes
    roof_us, roof_bytes = roofline_timing(ctx, gf, desc, prompt, args.kernel_iters)

    ctx.set_token_ids(0, prompt)
    for p, t in enumerate(prompt):
        ctx.forward(int(t), p, want_normx=False)
    pos = PROMPT_LEN
    for _ in range(args.warmup):
        ctx.step(pos, PENALTY, im_end, eos)
        pos += 1
    ctx.normx()  # drain
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.step(pos, PENALTY, im_end, eos)
        pos += 1
    ctx.sync()  # a step returns with its token while its forward still runs: the last one completes here
    dt = time.perf_counter() - t0
    ms_per_step = dt * 1000.0 / args.steps
    value = args.steps / dt
    t_first, t_last = PROMPT_LEN + args.warmup + 1, pos  # positions attended by the timed steps
    t_avg = 0.5 * (t_first + t_last)

    # the vocab kernel from HBM: launches back to back alternating between the
    # matrix and a device copy (twice 145 MB in flight, beyond the 256 MB
    # last-level cache), one pair of HIP events around them all
    vocab_ms = ctx.time_vocab(args.vocab_iters, pos, in_step=2)
    # every decode kernel, at the next position (attending pos + 1)
    kern = decode_kernels(ctx, gf, desc, vocab_ms, ms_per_step, pos + 1, args.kernel_iters)
    # a step's algorithmic bytes, however its kernels are grouped into launches
    kb = kernel_bytes(gf, desc, t_avg)
    step_bytes = (desc.n_layers * sum(kb[k] for k in ("qkv", "attn", "attn_out", "ffn_in", "ffn_out"))
                  + kb["final_norm"] + kb["vocab"])

    # device-fed steps at the host loop's positions, from the same state: the
    # prompt forwarded again and the same warm-up steps on the host, then
    # c2h_time_steps over the timed loop's positions
    ctx.set_token_ids(0, prompt)
    for p, t in enumerate(prompt):
        ctx.forward(int(t), p, want_normx=False)
    for p in range(PROMPT_LEN, PROMPT_LEN + args.warmup):
        ctx.step(p, PENALTY, im_end, eos)
    ctx.sync()
    pipelined_ms = ctx.time_steps(PROMPT_LEN + args.warmup, args.steps, PENALTY, im_end, eos)
    # and past them (positions pos .. pos + pipelined_iters - 1)
    pipelined_next_ms = ctx.time_steps(pos, args.pipelined_iters, PENALTY, im_end, eos)
    # In-step timing: a forward pass between launches streams the layer
    # weights, so the vocab rows come from HBM as they do inside a step.
    # Roofline timing: launches back to back alternating between the matrix
    # and a device copy (twice 145 MB in flight, beyond the 256 MB last-level
    # cache), so each reads its rows from HBM; one pair of HIP events around
    # them all.  In-step: a forward pass between launches, each launch
    # bracketed by its own events (which add its dispatch).
    vocab_step_ms = ctx.time_vocab(args.vocab_iters, pos, in_step=1)
    vocab_b2b_ms = ctx.time_vocab(args.vocab_iters, pos, in_step=0)
    vocab_gbs = VOCAB_BYTES / (vocab_ms * 1e-3) / 1e9
    # per-kernel floor of dependent launches in a graph (empty kernels); not
    # with C2H_NO_GRAPH=1 (eager runs, e.g. under a kernel-trace profiler)
    if os.environ.get("C2H_NO_GRAPH") == "1":
        floor_us, floor_by_grid = None, None
    else:
        floor_us = ctx.launch_floor(240, 256, 5)
        floor_by_grid = {g: round(ctx.launch_floor(240, g, 5), 3) for g in (1, 64, 256, 1024, 4096)}
    if args.copy_calib_mib:
        copy_calibration(ctx, args.copy_calib_mib)

    prefill = None if args.no_prefill else prefill_rate(ctx, desc, args.prefill_reps)
    lengths = [int(x) for x in args.long_context.split(",") if x]
    longctx = long_context(gf, im_end, eos, lengths) if lengths else None
    realf = None
    if not args.no_real_formats:
        rdir = tmpdir or tempfile.mkdtemp(prefix="c2slm_bench_")
        realf = real_formats(rdir, im_end, eos)
        if rdir != tmpdir:
            os.rmdir(rdir)

    qwen3 = None
    if not args.no_qwen3:
        rdir = tmpdir or tempfile.mkdtemp(prefix="c2slm_bench_")
        qwen3 = qwen3_decode(rdir, im_end, eos)
        if rdir != tmpdir:
            os.rmdir(rdir)
    fdots = None if args.no_float_dots else float_x_dots(ctx)
    micro = None if args.no_microbench else layer_microbench(ctx)

    achieved = roof_bytes / (roof_us * 1e-6) / 1e9
    dk = kern[ROOFLINE_KERNEL]

    base = None
    if not args.no_cpu_baseline:
        base = cpu_baseline(gf, prompt, args.steps, im_end, eos)

    line = {
        "metric": "decode tok/s @ Qwen2.5-0.5B-shape Q4_K_M, 1 GPU; achieved HBM GB/s",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot / fp32",
        "data": "synthetic (random-init GGUF v3, seed 20261201; random prompt ids)",
        "config": {"workload": f"full decode, Qwen2.5-0.5B shape (24L, 896, 14/2 heads, FFN 4864, vocab 151936), "
                               f"Q4_K/Q6_K/Q8_0, {PROMPT_LEN}-token prompt then greedy steps at positions "
                               f"{PROMPT_LEN + args.warmup}..{PROMPT_LEN + args.warmup + args.steps - 1}, "
                               f"repetition penalty {PENALTY}",
                   "batch": 1, "prompt_len": PROMPT_LEN, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(ROOFLINE_KERNEL),
                     "kernel": f"{ROOFLINE_KERNEL}: {dk['kernel']} (the layer kernel with the most bytes; "
                               f"{dk['share_of_step']:.0%} of the step)",
                     "bytes_per_launch": roof_bytes, "us_per_launch": round(roof_us, 3),
                     "timing": f"{args.kernel_iters} eager launches back to back over the 24 layers' weights, paced "
                               "by the GPU, one pair of HIP events on the context stream, on a fresh context after a "
                               "batched prefill of the prompt (the state `bench.py --only roofline` reproduces)"},
        "cpu_baseline": base,
        "extra": {"step": {"bytes": int(step_bytes), "gb_s": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                           "hbm_frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "attended_positions": [t_first, t_last]},
                  "decode_kernels": kern,
                  "vocab_from_hbm": {"ms": round(vocab_ms, 5), "gb_s": round(vocab_gbs, 1),
                                     "hbm_frac": round(vocab_gbs / HBM_PEAK_GBS, 4),
                                     "traffic": profiled_traffic("vocab")},
                  "layer_microbench": micro,
                  "vocab_ms_back_to_back": round(vocab_b2b_ms, 5),
                  "vocab_ms_in_step_events": round(vocab_step_ms, 5),
                  "launch_floor_us_per_kernel": None if floor_us is None else round(floor_us, 3),
                  "launch_floor_us_by_grid": floor_by_grid,
                  "pipelined_ms_per_step": round(pipelined_ms, 4),
                  "pipelined_tok_s": round(1000.0 / pipelined_ms, 1),
                  "pipelined_positions": [PROMPT_LEN + args.warmup, pos - 1],
                  "pipelined_next_tok_s": round(1000.0 / pipelined_next_ms, 1),
                  "pipelined_next_positions": [pos, pos + args.pipelined_iters - 1],
                  "prefill_512": prefill,
                  "long_context_decode": longctx,
                  "real_formats": realf,
                  "qwen3_1_7b_decode": qwen3,
                  "float_x_dots": fdots},
    }
    print(json.dumps(line))
    ctx.close()
    cleanup()


if __name__ == "__main__":
    main()
