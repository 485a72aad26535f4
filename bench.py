"""Benchmark: Llama-3-8B-shaped Q4 batch-1 greedy decode at 4k context on one
MI355X, plus the Q4 GEMV HBM roofline and the reference CPU path beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-traffic] [--gemv-only]

A step is one decode token: one pass of the hot path (embed, 32 layers of
normq / q-k-v GEMV / RoPE + fp16 KV attention / o GEMV / normq / SwiGLU GEMV /
down GEMV, then the head GEMV and greedy argmax) over synthetic random-init Q4
weights of the Llama-3-8B architecture. The prompt (random ids) is read first
so the timed tokens run with ~4k positions of KV cache. Prints one JSON line.
"""
import argparse
import ctypes
import json
import os
import shutil
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import sheep_amd as sa  # noqa: E402

HBM_PEAK_GBS = 8000.0
LLAMA = dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, n_ff=14336, n_vocab=128256,
             rope_theta=500000.0, rms_eps=1e-5, tied=False, qkv_bias=False, nbits=4, seed=1003)
N_CTX = 4096


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def scratch_dir():
    for d in (os.environ.get("SML_BENCH_DIR"), "/dev/shm", tempfile.gettempdir()):
        if d and os.path.isdir(d) and shutil.disk_usage(d).free > 12e9:
            return d
    return tempfile.gettempdir()


def gemv_roofline(rows, cols, iters=400, target_bytes=1.2e9, tmp=None):
    """Q4 GEMV over rotating copies (more bytes than the 256 MB MALL) timed
    with HIP events on the launch stream. Returns (avg_us, bytes_per_launch)."""
    p = os.path.join(tmp, f"gemv_{rows}x{cols}.ssf")
    if not os.path.exists(p):
        sa.synth_matrix(p, rows, cols, nbits=4, seed=1004)
    first = sa.Mat.from_file(p, "w")
    ncopy = max(2, int(target_bytes // first.bytes) + 1)
    mats = [first] + [sa.Mat.from_file(p, "w") for _ in range(ncopy - 1)]
    x = np.random.default_rng(0).standard_normal(cols).astype(np.float32)
    xd = sa.DevBuf.of(x)
    act = sa.Act(cols)
    sa.normq(xd, act)
    y = sa.DevBuf(rows * 4)
    arr = (sa.c_void_p * ncopy)(*[m.h for m in mats])
    ms = sa.c_float()
    lib = sa.lib()
    for _ in range(2):   # warm-up rounds
        assert lib.sml_hip_time_matvec(arr, ncopy, act.q.ptr, act.scale.ptr, act.sums.ptr, y.ptr, ncopy,
                                       sa.ctypes.byref(ms)) == 0
    trials = []
    for _ in range(5):
        assert lib.sml_hip_time_matvec(arr, ncopy, act.q.ptr, act.scale.ptr, act.sums.ptr, y.ptr, iters,
                                       sa.ctypes.byref(ms)) == 0
        trials.append(ms.value * 1000.0 / iters)
    for m in mats:
        m.free()
    return float(np.median(trials)), first.bytes


def read_ceiling(nbytes, iters=360, target_bytes=1.2e9, grid=2048):
    """What one streaming-read launch of nbytes takes from HBM: 16-byte
    nontemporal loads, grid-stride over `grid` 256-thread workgroups, over
    rotating buffers (> the 256 MB MALL), HIP events on the launch stream.
    The ceiling a single GEMV launch of that many bytes can approach."""
    nb = nbytes // 16 * 16
    nbuf = max(2, int(target_bytes // nb) + 1)
    bufs = [sa.DevBuf(nb) for _ in range(nbuf)]
    arr = (sa.c_void_p * nbuf)(*[b.ptr for b in bufs])
    ms = sa.c_float()
    lib = sa.lib()
    assert lib.sml_hip_time_read(arr, nbuf, nb, grid, 2 * nbuf, sa.ctypes.byref(ms)) == 0
    trials = []
    for _ in range(5):
        assert lib.sml_hip_time_read(arr, nbuf, nb, grid, iters, sa.ctypes.byref(ms)) == 0
        trials.append(ms.value * 1000.0 / iters)
    for b in bufs:
        b.free()
    return float(np.median(trials))


def gemv_size_sweep(tmp, cols=14336, rows_list=(4096, 8192, 16384, 32768, 65536)):
    """The Q4 GEMV and the streaming read at 34 .. 544 MB (rows x 14336),
    each over rotating copies: a line t = a + bytes / B through the points
    separates the fixed cost of a launch (a) from the steady-state rate (B)."""
    pts = []
    for rows in rows_list:
        us, nb = gemv_roofline(rows, cols, iters=max(40, 400 * 4096 // rows), tmp=tmp)
        rus = read_ceiling(nb, iters=max(40, 360 * 4096 // rows))
        pts.append({"rows": rows, "bytes": nb, "gemv_us": round(us, 3), "gemv_GB/s": round(nb / us / 1e3, 1),
                    "read_us": round(rus, 3), "read_GB/s": round(nb / rus / 1e3, 1)})
        log(f"sweep {rows}x{cols}: {pts[-1]}")
        os.remove(os.path.join(tmp, f"gemv_{rows}x{cols}.ssf"))
    x = np.array([p["bytes"] for p in pts], np.float64)
    out = {"points": pts}
    for key in ("gemv", "read"):
        y = np.array([p[f"{key}_us"] for p in pts], np.float64)
        slope, icpt = np.polyfit(x, y, 1)
        out[f"{key}_fixed_us"] = round(float(icpt), 3)
        out[f"{key}_steady_GB/s"] = round(1e-3 / float(slope), 1)
        out[f"{key}_steady_frac"] = round(1e-3 / float(slope) / HBM_PEAK_GBS, 4)
    return out


COPY_BYTES = 256 << 20
PROBE_LAUNCHES = 12


def pmc_probe(path):
    """Child of traffic(): the roofline GEMV on two copies of one matrix
    (PROBE_LAUNCHES launches) and a plain copy of COPY_BYTES (3 launches), so
    a counter pass sees both kernels in one process."""
    sa.init(0)
    a, b = sa.DevBuf(COPY_BYTES), sa.DevBuf(COPY_BYTES)
    for _ in range(3):
        if sa.lib().sml_hip_copy(b.ptr, a.ptr, COPY_BYTES) != 0:
            raise SystemExit("copy failed: " + sa.lib().sml_hip_last_error().decode())
    mats = [sa.Mat.from_file(path, "w") for _ in range(2)]
    rows, cols = mats[0].rows, mats[0].cols
    x = np.random.default_rng(0).standard_normal(cols).astype(np.float32)
    act = sa.Act(cols)
    sa.normq(sa.DevBuf.of(x), act)
    y = sa.DevBuf(rows * 4)
    for i in range(PROBE_LAUNCHES):
        sa.matvec(mats[i % 2], act, y)
    sa.sync()


def _counter_means(out_dir, counter):
    """Mean counter value per dispatch, by kernel name, from a rocprofv3
    counter-collection CSV."""
    import csv
    import glob
    files = glob.glob(os.path.join(out_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise RuntimeError(f"no counter_collection.csv under {out_dir}")
    vals = {}
    with open(files[0], newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return {k: float(np.mean(v)) for k, v in vals.items()}


def traffic(path, work):
    """HBM bytes per launch of the roofline GEMV from two rocprofv3 --pmc
    passes (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled by
    what the same counter reads for the copy kernel of known size. Returns
    (bytes, detail) or (None, reason)."""
    import subprocess
    rp = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3") else None)
    if rp is None:
        return None, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="pmc_", dir=work)
    env = dict(os.environ, TMPDIR=tmp)
    got = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = os.path.join(tmp, counter)
        cmd = ["timeout", "-s", "KILL", "90", rp, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "pmc",
               "--", sys.executable, os.path.abspath(__file__), "--pmc-probe", path]
        r = subprocess.run(cmd, cwd=tmp, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            return None, f"rocprofv3 --pmc {counter} exited {r.returncode}: {r.stdout[-300:]}"
        means = _counter_means(d, counter)
        gemv = [v for k, v in means.items() if k.startswith("sml_gemv_q4")]
        copy = [v for k, v in means.items() if k.startswith("sml_copy_stream")]
        if len(gemv) != 1 or len(copy) != 1:
            return None, f"{counter}: kernels seen {sorted(means)}"
        got[counter] = (gemv[0], copy[0])
    kib = COPY_BYTES / 1024.0
    f_fetch = kib / got["FETCH_SIZE"][1]
    f_write = kib / got["WRITE_SIZE"][1]
    t = got["FETCH_SIZE"][0] * 1024 * f_fetch + got["WRITE_SIZE"][0] * 1024 * f_write
    return t, {"fetch_kib": round(got["FETCH_SIZE"][0], 1), "write_kib": round(got["WRITE_SIZE"][0], 1),
               "copy_fetch_kib": round(got["FETCH_SIZE"][1], 1), "copy_write_kib": round(got["WRITE_SIZE"][1], 1),
               "copy_bytes": COPY_BYTES, "fetch_scale": round(f_fetch, 4), "write_scale": round(f_write, 4)}


def gemv_timeline(tmp, launches=24):
    """The roofline GEMV's timeline inside one cold launch (4096 x 14336 Q4,
    rotating copies beyond the MALL): per row block, the GPU clock (100 MHz)
    at entry, at its first weight word, when the first and the last pass's
    weights are all in, and at exit (sml_hip_gemv_timeline); per launch the
    spread over the 2048 blocks; medians over the launches, in us from the
    launch's first entry."""
    rows, cols = 4096, 14336
    p = os.path.join(tmp, "timeline_q4.ssf")
    sa.synth_matrix(p, rows, cols, nbits=4, seed=1004)
    first = sa.Mat.from_file(p, "w")
    mats = [first] + [sa.Mat.from_file(p, "w") for _ in range(int(6e8 // first.bytes))]
    x = np.random.default_rng(0).standard_normal(cols).astype(np.float32)
    act = sa.Act(cols)
    xd = sa.DevBuf.of(x)
    sa.normq(xd, act)
    y = sa.DevBuf(rows * 4)
    arr = (sa.c_void_p * len(mats))(*[m.h for m in mats])
    nb = rows // 8
    ts = np.zeros(nb * 5, np.uint64)
    lib = sa.lib()
    per = []
    for it in range(launches + 1):
        n = lib.sml_hip_gemv_timeline(arr, len(mats), act.q.ptr, act.scale.ptr, act.sums.ptr, y.ptr, len(mats),
                                      ts.ctypes.data, nb)
        if n != nb:
            raise RuntimeError(lib.sml_hip_last_error().decode())
        if it == 0:
            continue                                   # first call: the copies' pages warm in the TLB
        t = ts.reshape(nb, 5).astype(np.int64)
        t0 = t[:, 0].min()
        d = (t - t0) * 10 / 1000.0                     # us
        per.append({
            "span": float(d[:, 4].max()),
            "entry_p50": float(np.median(d[:, 0])), "entry_max": float(d[:, 0].max()),
            "first_word_latency_p50": float(np.median(d[:, 1] - d[:, 0])),
            "first_word_min": float(d[:, 1].min()), "first_word_p50": float(np.median(d[:, 1])),
            "pass1_all_in_p50": float(np.median(d[:, 2])), "last_weights_in_p50": float(np.median(d[:, 3])),
            "last_weights_in_max": float(d[:, 3].max()),
            "exit_p50": float(np.median(d[:, 4])), "exit_max": float(d[:, 4].max()),
        })
    for m in mats:
        m.free()
    os.remove(p)
    keys = per[0].keys()
    med = {k: round(float(np.median([q[k] for q in per])), 2) for k in keys}
    # the weights' bytes over the window from the first word anywhere to the last pass's last word
    rate = first.bytes / ((med["last_weights_in_max"] - med["first_word_min"]) * 1e-6) / 1e12
    return {"launches": len(per), "bytes": first.bytes, "median_us": med, "streaming_TB_per_s": round(rate, 2)}


def width_sweep(tmp, target_bytes=6e8, iters=200):
    """The fused GEMV at every SSF width and the GPTQ-style 4-bit layout, at
    4096 x 14336 and 14336 x 4096, over rotating copies (> the 256 MB MALL)."""
    from sheep_amd import gptq as gq
    out = {}
    x_cache = {}
    for rows, cols in ((4096, 14336), (14336, 4096)):
        for nb in (2, 3, 4, 5, 6, 8):
            p = os.path.join(tmp, f"sweep_q{nb}_{rows}x{cols}.ssf")
            sa.synth_matrix(p, rows, cols, nbits=nb, seed=1004)
            first = sa.Mat.from_file(p, "w")
            mats = [first] + [sa.Mat.from_file(p, "w") for _ in range(max(1, int(target_bytes // first.bytes)))]
            x = np.random.default_rng(0).standard_normal(cols).astype(np.float32)
            act = sa.Act(cols)
            sa.normq(sa.DevBuf.of(x), act)
            y = sa.DevBuf(rows * 4)
            arr = (sa.c_void_p * len(mats))(*[m.h for m in mats])
            ms = sa.c_float()
            lib = sa.lib()
            assert lib.sml_hip_time_matvec(arr, len(mats), act.q.ptr, act.scale.ptr, act.sums.ptr, y.ptr, len(mats),
                                           sa.ctypes.byref(ms)) == 0
            t = []
            for _ in range(3):
                assert lib.sml_hip_time_matvec(arr, len(mats), act.q.ptr, act.scale.ptr, act.sums.ptr, y.ptr, iters,
                                               sa.ctypes.byref(ms)) == 0
                t.append(ms.value * 1000.0 / iters)
            us = float(np.median(t))
            out[f"q{nb}_{rows}x{cols}"] = {"us": round(us, 3), "bytes": first.bytes,
                                           "GB/s": round(first.bytes / us / 1e3, 1)}
            for m in mats:
                m.free()
            os.remove(p)
        qw, qz, sc = gq.synth(rows, cols, seed=1004)
        first = gq.GptqMat(qw, qz, sc, rows, cols)
        mats = [first] + [gq.GptqMat(qw, qz, sc, rows, cols) for _ in range(max(1, int(target_bytes // first.bytes)))]
        xd = sa.DevBuf.of(np.random.default_rng(0).standard_normal(cols).astype(np.float32))
        y = sa.DevBuf(rows * 4)
        gq.time_matvec(mats, xd, y, len(mats))
        us = float(np.median([gq.time_matvec(mats, xd, y, iters) * 1000.0 / iters for _ in range(3)]))
        out[f"gptq4_{rows}x{cols}"] = {"us": round(us, 3), "bytes": first.bytes, "GB/s": round(first.bytes / us / 1e3, 1)}
        for m in mats:
            m.free()
    return out


def moe_layer(tmp, T=16, iters=50):
    """A Mixtral-shaped MoE FFN layer (hidden 4096, 8 experts of 14336 SwiGLU
    Q4, top-2 softmax over the chosen, f32 router) on T tokens of N(0,1)
    input: time per step and the bytes of the experts the step touches, with
    the expert inputs quantized per 32 (the stepped moe_ffn's regime) and per
    256 (moe_ffn_batch's in the batched regimes)."""
    p = os.path.join(tmp, "mixtral_layer.ssf")
    sa.synth_model(p, n_layer=1, n_embd=4096, n_head=32, n_head_kv=8, n_ff=14336, n_vocab=1024, n_expert=8,
                   n_expert_used=2, moe_flags=1, rope_theta=1e6, seed=1005)
    moe = sa.MoE(p, 0, 16)
    x = sa.DevBuf.of(np.random.default_rng(1005).standard_normal((T, 4096)).astype(np.float32))
    out = sa.DevBuf(T * 4096 * 4)
    res = {"tokens": T}
    for name, sb in (("per32", False), ("per256", True)):
        moe.regime(sb)
        moe.time(x, T, out, 3)
        ms, cnt = moe.time(x, T, out, iters)
        us = ms * 1000.0 / iters
        touched = int((cnt > 0).sum())
        b = touched * moe.expert_bytes + moe.nexp * 4096 * 4
        res.update({"experts_touched": touched, "tokens_per_expert": cnt.tolist(), "bytes_per_step": b})
        res[name] = {"us_per_step": round(us, 2), "GB/s": round(b / us / 1e3, 1)}
    moe.free()
    res["path"] = p               # kept for the CPU baseline's MoE leg
    return res


QWEN = dict(n_layer=28, n_embd=1536, n_head=12, n_head_kv=2, n_ff=8960, n_vocab=151936, rope_theta=1e6,
            rms_eps=1e-6, qkv_bias=True, tied=True, random_perm=False, nbits=4, seed=1002)


def qwen_decode(tmp, prompt_len=2048, steps=64):
    """The Qwen2.5-1.5B-shaped decoder (28 layers, hidden 1536, FFN 8960,
    12/2 heads, tied 151936-token head, q/k/v bias, identity permutations):
    a 2048-id prompt read a token at a time, then 64 greedy tokens timed as
    one generate call."""
    path = os.path.join(tmp, "qwen25_1p5b_q4.ssf")
    sa.synth_model(path, n_ctx_train=4096, **QWEN)
    dec = sa.Decoder(path, n_ctx=prompt_len + steps + 8)
    try:
        ids = np.random.default_rng(1002).integers(0, QWEN["n_vocab"], prompt_len).astype(np.int32)
        t0 = time.perf_counter()
        tok = int(np.argmax(dec.prefill(ids, 0, QWEN["n_vocab"])))
        t_prompt = time.perf_counter() - t0
        dec.generate(tok, prompt_len, 4)                     # warm-up (graph capture)
        sa.sync()
        t0 = time.perf_counter()
        dec.generate(tok, prompt_len, steps)
        sa.sync()
        dt = time.perf_counter() - t0
        wbytes = dec.weight_bytes()
    finally:
        dec.close()
        os.remove(path)
    return {"tokens": steps, "positions": f"{prompt_len}..{prompt_len + steps - 1}",
            "prompt_tokens_per_s": round(prompt_len / t_prompt, 1),
            "tokens_per_s": round(steps / dt, 1), "weight_bytes_per_token": wbytes,
            "roofline_tokens_per_s_weights_only": round(HBM_PEAK_GBS * 1e9 / wbytes, 1),
            "frac_of_weights_roofline": round(steps / dt / (HBM_PEAK_GBS * 1e9 / wbytes), 4)}


def exact_decode(path, ids, warmup, steps):
    """The token-identical path: the same Llama-3-8B-shaped file opened in
    exact mode (every kernel in the reference CPU engine's float order, so
    each step's logits equal its sml_forward bit for bit), the same prompt
    read exactly (batched: 64-position chunks through the reference-order
    GEMM and attention, equal to stepping it bit for bit), then `warmup`
    untimed and `steps` timed greedy tokens at the fast line's positions."""
    dec = sa.Decoder(path, n_ctx=N_CTX, exact=True)
    try:
        if not dec.exact:
            raise RuntimeError("exact mode did not open")
        t0 = time.perf_counter()
        lg = dec.prefill(ids, 0, LLAMA["n_vocab"])
        t_prompt = time.perf_counter() - t0
        pos = len(ids)
        warm = dec.generate(int(np.argmax(lg)), pos, warmup)
        tok, pos = int(warm[-1]), pos + warmup
        sa.sync()
        t1 = time.perf_counter()
        out = dec.generate(tok, pos, steps)
        sa.sync()
        dt = time.perf_counter() - t1
        ev_ms = dec.last_ms()
        wbytes = dec.weight_bytes()
    finally:
        dec.close()
    tps = steps / dt
    return {"positions": f"{pos}..{pos + steps - 1}", "tokens_per_s": round(tps, 2),
            "ms_per_step": round(dt * 1e3 / steps, 4), "gpu_event_ms": round(ev_ms, 3),
            "frac_of_weights_roofline": round(tps / (HBM_PEAK_GBS * 1e9 / wbytes), 4),
            "prompt": {"tokens": len(ids), "level": 1, "s": round(t_prompt, 3),
                       "tokens_per_s": round(len(ids) / t_prompt, 1)},
            "first_tokens": [int(t) for t in out[:8]]}


def small_gemm(tmp, M=16, iters=60):
    """The 16-row small-M GEMMs of the batched step over rotating copies:
    SwiGLU gate+up 2 x 14336 x 4096, 4096 x 4096 and 4096 x 14336, with
    seeded int8 activation rows, for per-32 and per-256 activations (the
    per-256 scale repeats over each superblock's 8 groups). Returns µs per
    launch (best of 3) and the weight bytes' rate."""
    rng = np.random.default_rng(1005)
    out = {}
    for rows, cols, sw, n in [(14336, 4096, True, 8), (4096, 4096, False, 24), (6144, 4096, False, 24),
                              (4096, 14336, False, 16)]:
        p = os.path.join(tmp, f"gemm_{rows}x{cols}.ssf")
        sa.synth_matrix(p, rows, cols, nbits=4, seed=1005)
        mats = [sa.Mat.from_file(p, "w") for _ in range(n * (2 if sw else 1))]
        q = sa.DevBuf.of(rng.integers(-127, 128, M * cols).astype(np.int8))
        s32 = (np.abs(rng.standard_normal(M * cols // 32)) * 0.01).astype(np.float32)
        s = sa.DevBuf.of(s32)
        s256 = sa.DevBuf.of(np.repeat(s32.reshape(-1, 8)[:, :1], 8, axis=1).reshape(-1))
        u = sa.DevBuf.of(rng.integers(-2000, 2000, M * cols // 32).astype(np.int32))
        y = sa.DevBuf(M * rows * 4)
        nbytes = mats[0].bytes * (2 if sw else 1)
        res = {"rows_m": M}
        for name, sb, sc in (("per32", False, s), ("per256", True, s256)):
            if sw:
                fn = lambda i: sa.gemm_swiglu(mats[2 * (i % n)], mats[2 * (i % n) + 1], q, sc, u, M, y, per256=sb)
            else:
                fn = lambda i: sa.gemm(mats[i % n], q, sc, u, M, y, per256=sb)
            for i in range(4):
                fn(i)
            sa.sync()
            best = 1e9
            for _ in range(3):
                t0 = time.perf_counter()
                for i in range(iters):
                    fn(i)
                sa.sync()
                best = min(best, (time.perf_counter() - t0) / iters * 1e6)
            res[name] = {"us": round(best, 2), "GB/s": round(nbytes / best / 1e3, 1)}
        out[f"{'swiglu_2x' if sw else ''}{rows}x{cols}"] = res
        for m in mats:
            m.free()
        os.remove(p)
    return out


def batched_decode(dec, n_vocab, ns=16, steps=20, pos0=1024):
    """Aggregate tokens/s of ns sequences stepped together (sml_gpu_step_multi)
    at positions pos0.. of their own KV slots, in the default regime (per-256
    activations above two sequences) and the per-32 one."""
    dec.slots(ns)
    res = {"sequences": ns}
    for name, env in (("per256", None), ("per32", "16")):
        if env:
            os.environ["SML_MULTI_EXACT_MAX"] = env
        try:
            for b in range(ns):
                dec.prefill_slot(b, (np.arange(8, dtype=np.int32) * 7 + b) % n_vocab, pos0 - 8, n_vocab)
            toks = list(range(1, ns + 1))
            dec.step_multi(toks, [pos0] * ns, list(range(ns)), n_vocab)
            sa.sync()
            t0 = time.perf_counter()
            gpu_ms = 0.0
            for i in range(steps):
                dec.step_multi(toks, [pos0 + 1 + i] * ns, list(range(ns)), n_vocab)
                gpu_ms += dec.last_ms()
            dt = time.perf_counter() - t0
        finally:
            os.environ.pop("SML_MULTI_EXACT_MAX", None)
        # wall time per step includes copying every sequence's logits to the
        # host (16 x 128256 floats); the GPU time is the step's kernels alone
        res[name] = {"ms_per_step": round(dt / steps * 1e3, 3), "tokens_per_s": round(ns * steps / dt, 1),
                     "gpu_ms_per_step": round(gpu_ms / steps, 3),
                     "gpu_tokens_per_s": round(ns * steps / (gpu_ms / 1e3), 1),
                     "positions": f"{pos0 + 1}..{pos0 + steps}"}
    return res


def ingest_leg(rows=4096, cols=14336, trials=3):
    """The GPTQ-4 tensor of the width sweep (group 128, seed 1004)
    re-quantized into SSF Q4 on the device: unpack to fp16, column order,
    grid search, two-level fields, field search, codes and planes. GPU time
    from HIP events around the kernels, best of `trials`."""
    from sheep_amd import gptq as gq, ingest
    qw, qz, sc = gq.synth(rows, cols, seed=1004)
    t = {"qweight": qw, "qzeros": qz, "scales": sc}
    qc = {"bits": 4, "group_size": 128}
    ingest.ingest_gptq(t, qc)                    # warm-up
    best, wall = 1e9, 1e9
    for _ in range(trials):
        sa.sync()
        t0 = time.perf_counter()
        r = ingest.ingest_gptq(t, qc)
        sa.sync()
        wall = min(wall, time.perf_counter() - t0)
        best = min(best, r.ms)
    n = rows * cols
    return {"tensor": f"GPTQ-4 {rows}x{cols} group 128 -> SSF Q4", "weights": n, "gpu_ms": round(best, 3),
            "weights_per_s": round(n / (best * 1e-3), 1), "wall_ms_with_uploads": round(wall * 1e3, 2)}


def host_cpu():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "usable": len(os.sched_getaffinity(0)), "cpu": model}


def cpu_leg(args):
    """One CPU-baseline measurement in its own process, pinned to CPUs
    0..T-1 (the reference's pool threads inherit the affinity). Prints one
    JSON object."""
    kind, threads = args[0], int(args[1])
    avail = sorted(os.sched_getaffinity(0))
    os.sched_setaffinity(0, avail[:threads])
    from oracle import bind as ob
    if not ob.have_ref():
        print(json.dumps({"error": "oracle/_ref/libsmlref.so not built"}))
        return
    if kind == "decode":
        # positions pos0 + 1 .. end, cycled until the budget is spent (a
        # revisited position overwrites its cache row and attends to the
        # rows before it, the same work as the first visit)
        path, pos0, budget, end = args[2], int(args[3]), float(args[4]), int(args[5])
        span = end - pos0
        m = ob.RefModel(path, end + 1, threads=threads)
        tok = 1
        m.forward(tok, pos0)                     # warm-up token
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget or n < 2:
            tok = int(np.argmax(m.forward(tok, pos0 + 1 + n % span)))
            n += 1
        dt = time.perf_counter() - t0
        m.close()
        cycled = f", cycled {n / span:.1f} times" if n > span else ""
        print(json.dumps({"tokens": n, "s": round(dt, 3), "tokens_per_s": round(n / dt, 3),
                          "positions": f"{pos0 + 1}..{pos0 + min(n, span)}{cycled}"}))
    elif kind == "gemv":
        from sheep_amd.ssf import SSF
        path, ncopy = args[2], int(args[3])
        t = SSF(path)["w"]
        cols, rows = t.cols, t.rows
        copies = []
        for _ in range(ncopy):
            pl = [np.array(p) for p in t.planes()] + [np.zeros(16, np.uint8)] * (3 - len(t.planes()))
            copies.append((pl, np.array(t.sd), np.array(t.sq), np.array(t.md), np.array(t.mq)))
        V = ctypes.c_void_p
        planes = (V * (3 * ncopy))(*[p.ctypes.data for c in copies for p in c[0]])
        arrs = [(V * ncopy)(*[c[i].ctypes.data for c in copies]) for i in range(1, 5)]
        x = np.random.default_rng(0).standard_normal(cols).astype(np.float32)
        r = ob.ref()
        r.ref_time_matvec.restype = ctypes.c_double
        r.ref_time_matvec.argtypes = [V] * 5 + [ctypes.c_int] * 4 + [V, ctypes.c_int, ctypes.c_int]
        nb = t.planes_bytes if hasattr(t, "planes_bytes") else None
        sec = r.ref_time_matvec(planes, arrs[0], arrs[1], arrs[2], arrs[3], ncopy, rows, cols, t.nbits,
                                x.ctypes.data, threads, 12)
        print(json.dumps({"us": round(sec * 1e6, 1), "rows": rows, "cols": cols, "nbits": t.nbits}))
    elif kind == "ingest":
        # the reference quantizer's fused C searches (sml-quant.c, OpenMP over
        # rows) on a row slice of the same float16 copy: the grid, then the
        # field search on its two-level fields
        from sheep_amd import gptq as gq
        rows, cols, sample = int(args[2]), int(args[3]), int(args[4])
        qw, qz, sc = gq.synth(rows, cols, seed=1004)
        w = ob.unpack_dequant_f16(qw, qz, sc, None, rows, cols, 4, 128, 1)[:sample]
        rq = ob.refq()
        t0 = time.perf_counter()
        mins, steps = ob.asym_grid(w, 32, 4, lib=rq)
        t1 = time.perf_counter()
        d16, q8, _ = ob.two_level(steps, 8, signed=False)
        md16, mq8, _ = ob.two_level(mins, 8, signed=True)
        dv = np.repeat(d16.view(np.float16).astype(np.float32), 8, axis=1)
        dm = np.repeat(md16.view(np.float16).astype(np.float32), 8, axis=1)
        t2 = time.perf_counter()
        ob.field_search(w, dv, dm, q8, mq8, 32, 15, lib=rq)
        t3 = time.perf_counter()
        n = sample * cols
        print(json.dumps({"rows_sampled": sample, "weights": n, "grid_s": round(t1 - t0, 3),
                          "field_s": round(t3 - t2, 3),
                          "weights_per_s": round(n / ((t1 - t0) + (t3 - t2)), 1)}))
    elif kind == "moe":
        path, regime, steps = args[2], args[3], int(args[4])
        if regime == "exact":
            os.environ["SML_MULTI"] = "exact"
        ns = 16
        m = ob.RefMulti(path, 64, ns, threads=threads)
        toks, pos = list(range(1, ns + 1)), [0] * ns
        m.step(toks, pos)                        # warm-up step
        t0 = time.perf_counter()
        for s in range(steps):
            m.step(toks, [s + 1] * ns)
        dt = time.perf_counter() - t0
        m.close()
        print(json.dumps({"slots": ns, "steps": steps, "ms_per_step": round(dt / steps * 1e3, 2),
                          "tokens_per_s": round(ns * steps / dt, 2), "regime": regime}))


def run_cpu_leg(*args, timeout=300):
    """A CPU leg in a child process (its own pinning and environment)."""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-leg"] + [str(a) for a in args]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=timeout,
                       env=dict(os.environ, OMP_NUM_THREADS=str(args[1])))
    try:
        return json.loads(r.stdout.strip().splitlines()[-1])
    except (ValueError, IndexError):
        return {"error": f"exit {r.returncode}: {r.stderr[-300:]}"}


def cpu_baseline(path, pos0, moe_path, gemv_paths, budget_s=10.0):
    """The reference's own CPU path (sml-kernel.c kernels on sml-pool threads,
    compiled from its sources into oracle/_ref) on the same files, on this
    host's cores, each leg pinned to its first T CPUs:
    - decode (sml_forward) at the GPU line's positions (pos0 + 1 .. the
      context's last, cycled; the cache rows before them are left as
      allocated, which costs the same reads),
      T = every usable CPU (the value), with the T sweep and a short-context line;
    - the single-GEMV workloads (sml_quantize_act + the width's kernels over row
      chunks of 32, rotating over copies larger than the LLC);
    - the MoE layer through sml_forward_multi with 16 slots, both regimes."""
    host = host_cpu()
    tmax = host["usable"]
    sweep_t = [t for t in (1, 8, 16, 32) if t < tmax] + [tmax]
    out = {"kind": "reference", "unit": "tokens/s", "host": host}
    sweep = {}
    for t in sweep_t:
        sweep[str(t)] = run_cpu_leg("decode", t, path, pos0, budget_s if t == tmax else budget_s / 2, N_CTX - 1)
        log(f"cpu decode T={t}: {sweep[str(t)]}")
    best = max(sweep, key=lambda k: sweep[k].get("tokens_per_s", 0))
    out["value"] = sweep[str(tmax)].get("tokens_per_s")
    out["cores"] = tmax
    out["threads_sweep"] = sweep
    out["best_threads"] = int(best)
    out["short_context"] = run_cpu_leg("decode", tmax, path, 1, budget_s / 2, 2001)
    out["sample"] = (f"{sweep[str(tmax)].get('tokens')} greedy tokens of the same Llama-3-8B-shaped Q4 file at "
                     f"positions {sweep[str(tmax)].get('positions')} (the GPU line's), sml_forward on {tmax} pool "
                     f"threads pinned to CPUs 0..{tmax - 1}; T sweep {sweep_t}; {host['cpu']}, "
                     f"{host['nproc']} CPUs ({tmax} usable, one socket)")
    g = {}
    for name, p in gemv_paths.items():
        g[name] = run_cpu_leg("gemv", tmax, p, 4)
        if "us" in g[name]:
            g[name]["GB/s"] = round(os.path.getsize(p) / g[name]["us"] / 1e3, 1)
        log(f"cpu gemv {name}: {g[name]}")
    out["gemv"] = g
    if moe_path:
        out["moe_16_slots"] = {r: run_cpu_leg("moe", tmax, moe_path, r, 6) for r in ("default", "exact")}
        log(f"cpu moe: {out['moe_16_slots']}")
    from oracle import bind as ob
    if ob.have_refq():
        out["ingest"] = run_cpu_leg("ingest", tmax, 4096, 14336, 512)
        log(f"cpu ingest searches: {out['ingest']}")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gemv-only", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 --pmc passes")
    ap.add_argument("--no-extra", action="store_true", help="skip the batched, MoE and width-sweep lines")
    ap.add_argument("--no-exact", action="store_true", help="skip the exact-mode decode leg")
    ap.add_argument("--pmc-probe", metavar="SSF", help=argparse.SUPPRESS)
    ap.add_argument("--cpu-leg", nargs="+", help=argparse.SUPPRESS)
    ap.add_argument("--decode-trace", metavar="MODEL", choices=("llama", "qwen"),
                    help="only decode the last --steps positions with direct launches (run under rocprofv3)")
    ap.add_argument("--exact", action="store_true",
                    help="with --decode-trace or --prompt-only: open the decoder in exact mode (the reference's "
                         "float order)")
    ap.add_argument("--trace-summary", metavar="DIR", help="per-kernel table of a --decode-trace kernel trace")
    ap.add_argument("--small-gemm", action="store_true", help="only time the 16-row small-M GEMMs")
    ap.add_argument("--gemv-sweep", action="store_true",
                    help="only the Q4 GEMV and streaming read at 34..544 MB (fixed cost vs steady rate)")
    ap.add_argument("--ingest", action="store_true", help="only re-quantize the GPTQ-4 4096 x 14336 tensor")
    ap.add_argument("--gemv-timeline", action="store_true",
                    help="only the roofline GEMV's in-kernel timeline (entry, first weight word, last, exit)")
    ap.add_argument("--batched-trace", action="store_true",
                    help="only the 16-sequence batched step, --steps steps after a marker copy, direct launches "
                         "(run under rocprofv3; summarise with --trace-summary)")
    ap.add_argument("--split", type=int, nargs="*", metavar="K",
                    help="only the layer split: a 1024-id prompt (levels 2 and 1) and 16 decode steps with K of "
                         "the 32 Llama layers' matrices in HBM (default K: 32 24 16)")
    ap.add_argument("--widths", action="store_true",
                    help="only the GEMV at every SSF width and the GPTQ-4 layout (4096x14336, 14336x4096)")
    ap.add_argument("--keep", action="store_true", help="keep the generated model file")
    ap.add_argument("--prompt", type=int, default=0, help="prompt length (default: fill the 4096 context)")
    ap.add_argument("--prompt-only", type=int, metavar="LEVEL", default=-1,
                    help="only read the Llama-3-8B-shaped prompt at this prompt level (0, 1 or 2)")
    a = ap.parse_args()
    if a.cpu_leg:
        cpu_leg(a.cpu_leg)
        return
    if a.trace_summary:
        print(trace_summary(a.trace_summary, a.steps))
        return
    if a.pmc_probe:
        pmc_probe(a.pmc_probe)
        return
    if a.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {a.gpus} is not supported (this build has no "
              f"multi-GPU path)", file=sys.stderr)
        sys.exit(2)
    sa.init(0)
    tmp = scratch_dir()
    work = tempfile.mkdtemp(prefix="smlbench_", dir=tmp)
    try:
        if a.small_gemm:
            res = {"small_m_gemm": small_gemm(work)}
        elif a.gemv_sweep:
            res = {"gemv_size_sweep": gemv_size_sweep(work)}
        elif a.ingest:
            res = {"ingest": ingest_leg()}
        elif a.gemv_timeline:
            res = {"gemv_timeline": gemv_timeline(work)}
        elif a.widths:
            res = {"width_sweep": width_sweep(work, iters=50)}
        elif a.decode_trace:
            res = {"decode_trace": decode_trace(work, a.decode_trace, a.steps, a.exact)}
        elif a.split is not None:
            res = {"split": split_leg(work, a.split or [32, 24, 16])}
        elif a.batched_trace:
            res = {"batched_trace": batched_trace(work, a.steps)}
        elif a.prompt_only >= 0:
            res = {"prompt_reading": prompt_only(work, a.prompt_only, a.prompt if a.prompt > 0 else 3960, a.exact)}
        else:
            res = run(a, work)
    finally:
        if not a.keep:
            shutil.rmtree(work, ignore_errors=True)
    print(json.dumps(res), flush=True)


def decode_trace(work, model="llama", steps=32, exact=False):
    """For a kernel trace of the timed decode region only: the Llama-3-8B-
    (or Qwen2.5-1.5B-) shaped file opened with direct launches (SML_GRAPH=0:
    the tracer sees each kernel), its prompt read at level 1 (exact mode: a
    token at a time) so the cache holds N_CTX - steps positions, then a
    16-byte copy (sml_copy_stream, the marker) and `steps` greedy tokens at
    the last positions of the context."""
    os.environ["SML_GRAPH"] = "0"
    spec = LLAMA if model == "llama" else QWEN
    path = os.path.join(work, f"{model}_trace.ssf")
    sa.synth_model(path, n_ctx_train=N_CTX, **spec)
    dec = sa.Decoder(path, n_ctx=N_CTX, exact=exact)
    try:
        n = N_CTX - steps
        ids = np.random.default_rng(1003).integers(0, spec["n_vocab"], n).astype(np.int32)
        t0 = time.perf_counter()
        lg = dec.prefill(ids, 0, spec["n_vocab"])
        log(f"prompt of {n} ids read in {time.perf_counter() - t0:.1f} s")
        a, b = sa.DevBuf(64), sa.DevBuf(64)
        assert sa.lib().sml_hip_copy(b.ptr, a.ptr, 16) == 0
        sa.sync()
        dec.generate(int(np.argmax(lg)), n, steps)
    finally:
        dec.close()
    return {"model": model, "exact": exact, "decode_positions": f"{N_CTX - steps}..{N_CTX - 1}", "steps": steps}


def split_leg(work, ks, n=1024, steps=16):
    """The Llama-3-8B-shaped file opened with gpu_layers = k for each k: the
    other layers' matrices are streamed from pinned host memory ahead of
    each use. A prompt of n ids at levels 2 and 1 (after a 64-id warm-up
    read), then `steps` greedy steps from position n + 3; wall time around
    each (a split model launches directly)."""
    path = os.path.join(work, "llama_split.ssf")
    sa.synth_model(path, n_ctx_train=N_CTX, **LLAMA)
    V = LLAMA["n_vocab"]
    ids = (np.arange(n, dtype=np.int32) * 7 + 3) % V
    out = {}
    for k in ks:
        dec = sa.Decoder(path, n_ctx=N_CTX, gpu_layers=k)
        try:
            r = {"layers_in_hbm": dec.gpu_layers, "of": dec.n_layer}
            for lvl in (2, 1):
                dec.prompt_mode(lvl)
                dec.prefill(ids[:64], 0, V)
                sa.sync()
                t = time.perf_counter()
                lg = dec.prefill(ids, 0, V)
                dt = time.perf_counter() - t
                r[f"prompt_level{lvl}"] = {"tokens": n, "ms": round(dt * 1e3, 1), "tokens_per_s": round(n / dt, 1)}
            for i in range(3):
                lg = dec.step(int(np.argmax(lg)), n + i, V)
            sa.sync()
            t = time.perf_counter()
            for i in range(steps):
                lg = dec.step(int(np.argmax(lg)), n + 3 + i, V)
            dt = time.perf_counter() - t
            r["decode"] = {"steps": steps, "ms_per_token": round(dt / steps * 1e3, 2),
                           "tokens_per_s": round(steps / dt, 1)}
            out[str(k)] = r
            log(f"split {k}: {r}")
        finally:
            dec.close()
    return out


def batched_trace(work, steps=10, ns=16, pos0=1024):
    """For a kernel trace of the 16-sequence batched step (per-256 regime):
    the Llama-3-8B-shaped file with direct launches (SML_GRAPH=0), ns slots
    with 8-id prompts ending at pos0 - 1, one untimed step, a 16-byte copy
    (sml_copy_stream, the marker), then `steps` steps at positions pos0 + 1..
    (the bench line's batched_decode leg, launched one kernel at a time)."""
    os.environ["SML_GRAPH"] = "0"
    path = os.path.join(work, "llama_batched_trace.ssf")
    sa.synth_model(path, n_ctx_train=N_CTX, **LLAMA)
    V = LLAMA["n_vocab"]
    dec = sa.Decoder(path, n_ctx=N_CTX)
    try:
        dec.slots(ns)
        for b in range(ns):
            dec.prefill_slot(b, (np.arange(8, dtype=np.int32) * 7 + b) % V, pos0 - 8, V)
        toks = list(range(1, ns + 1))
        dec.step_multi(toks, [pos0] * ns, list(range(ns)), V)
        a, b = sa.DevBuf(64), sa.DevBuf(64)
        assert sa.lib().sml_hip_copy(b.ptr, a.ptr, 16) == 0
        sa.sync()
        for i in range(steps):
            dec.step_multi(toks, [pos0 + 1 + i] * ns, list(range(ns)), V)
        sa.sync()
    finally:
        dec.close()
    return {"sequences": ns, "positions": f"{pos0 + 1}..{pos0 + steps}", "steps": steps}


def trace_summary(out_dir, steps):
    """Per-kernel statistics of the dispatches after the last marker copy in
    a rocprofv3 --kernel-trace CSV, as a markdown table (per decode token)."""
    import csv
    import glob
    files = glob.glob(os.path.join(out_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_trace.csv under {out_dir}")
    rows = []
    with open(files[0], newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    last = max(i for i, r in enumerate(rows) if r[2].startswith("sml_copy_stream"))
    dec = rows[last + 1:]
    stats = {}
    for s, e, name in dec:
        stats.setdefault(name, []).append((e - s) / 1e3)
    span = (dec[-1][1] - dec[0][0]) / 1e3
    busy = sum(v for vs in stats.values() for v in vs)
    lines = [f"Dispatches after the marker: {len(dec)} over {steps} tokens; span {span:.1f} us "
             f"({span / steps:.1f} us per token), kernels busy {busy / steps:.1f} us per token.", "",
             "| kernel | per token | mean us | min us | max us | us per token | share |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for name, v in sorted(stats.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{name}` | {len(v) / steps:g} | {np.mean(v):.2f} | {np.min(v):.2f} | {np.max(v):.2f} | "
                     f"{sum(v) / steps:.1f} | {sum(v) / busy:.1%} |")
    return "\n".join(lines)


def prompt_only(work, level, n, exact=False):
    """The Llama-3-8B-shaped file's prompt of n ids read once at one prompt
    level (exact: opened in exact mode, where level 1 is the reference-order
    batched prompt)."""
    path = os.path.join(work, "llama3_8b_q4.ssf")
    sa.synth_model(path, n_ctx_train=N_CTX, **LLAMA)
    dec = sa.Decoder(path, n_ctx=N_CTX, exact=exact)
    try:
        ids = np.random.default_rng(1003).integers(0, LLAMA["n_vocab"], n).astype(np.int32)
        dec.prompt_mode(level)
        dec.prefill(ids[:64], 0, LLAMA["n_vocab"])       # untimed: allocates the batched buffers
        sa.sync()
        t0 = time.perf_counter()
        dec.prefill(ids, 0, LLAMA["n_vocab"])
        dt = time.perf_counter() - t0
    finally:
        dec.close()
    return {"level": level, "exact": exact, "tokens": n, "s": round(dt, 3), "tokens_per_s": round(n / dt, 1)}


def run(a, work):
    t0 = time.perf_counter()
    g_us, g_bytes = gemv_roofline(4096, 14336, tmp=work)
    g2_us, g2_bytes = gemv_roofline(14336, 4096, tmp=work)
    g1_us, g1_bytes = gemv_roofline(8960, 1536, tmp=work)
    gbs = g_bytes / (g_us * 1e-6) / 1e9
    log(f"gemv q4 4096x14336: {g_us:.2f} us, {gbs:.0f} GB/s; 14336x4096: {g2_us:.2f} us, "
        f"{g2_bytes / g2_us / 1e3:.0f} GB/s; 8960x1536: {g1_us:.2f} us, {g1_bytes / g1_us / 1e3:.0f} GB/s "
        f"({time.perf_counter() - t0:.1f}s)")
    roof = {"bound": "hbm", "kernel": "sml_gemv_q4 (4096 rows x 14336 cols, Q4)",
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None, "avg_us": round(g_us, 3), "bytes_per_launch": g_bytes}
    r_us = read_ceiling(g_bytes)
    roof["read_ceiling"] = {"us": round(r_us, 3), "GB/s": round(g_bytes / r_us / 1e3, 1),
                            "frac": round(g_bytes / r_us / 1e3 / HBM_PEAK_GBS, 4),
                            "gemv_over_read": round(r_us / g_us, 4)}
    log(f"streaming read of the same {g_bytes} bytes: {r_us:.2f} us; the GEMV runs at {r_us / g_us:.1%} of it")
    if not a.no_traffic:
        t1 = time.perf_counter()
        tb, detail = traffic(os.path.join(work, "gemv_4096x14336.ssf"), work)
        roof["traffic"] = None if tb is None else int(round(tb))
        roof["traffic_detail"] = detail
        log(f"pmc traffic: {tb} bytes/launch vs {g_bytes} algorithmic; {detail} ({time.perf_counter() - t1:.1f}s)")
    gemv = {"4096x14336": {"us": round(g_us, 3), "GB/s": round(gbs, 1)},
            "14336x4096": {"us": round(g2_us, 3), "GB/s": round(g2_bytes / g2_us / 1e3, 1)},
            "8960x1536": {"us": round(g1_us, 3), "GB/s": round(g1_bytes / g1_us / 1e3, 1)}}
    if a.gemv_only:
        return {"metric": "Q4 GEMV HBM GB/s", "value": round(gbs, 1), "unit": "GB/s", "roofline": roof, "gemv_q4": gemv}

    path = os.path.join(work, "llama3_8b_q4.ssf")
    t1 = time.perf_counter()
    sa.synth_model(path, n_ctx_train=N_CTX, **LLAMA)
    log(f"synthetic Llama-3-8B-shaped Q4 file: {os.path.getsize(path) / 1e9:.2f} GB ({time.perf_counter() - t1:.1f}s)")
    K, W = a.steps, a.warmup
    prompt_len = a.prompt if a.prompt > 0 else N_CTX - K - W
    if prompt_len < 1 or prompt_len + K + W > N_CTX:
        raise SystemExit("steps + warmup must stay below the 4096-position context")
    t1 = time.perf_counter()
    dec = sa.Decoder(path, n_ctx=N_CTX)
    wbytes = dec.weight_bytes()
    log(f"loaded on the GPU in {time.perf_counter() - t1:.1f}s; {wbytes / 1e9:.4f} GB of weights per token")
    rng = np.random.default_rng(1003)
    ids = rng.integers(0, LLAMA["n_vocab"], prompt_len).astype(np.int32)
    prompt = {"tokens": prompt_len}
    if not a.no_extra:
        # the other prompt levels first (each rewrites the same cache
        # positions); the default level last, so decode starts from its cache.
        # An untimed short prompt first allocates the batched buffers.
        dec.prompt_mode(2)
        dec.prefill(ids[:64], 0, LLAMA["n_vocab"])
        for lvl, n in ((2, prompt_len), (0, min(prompt_len, 256))):
            dec.prompt_mode(lvl)
            sa.sync()
            t1 = time.perf_counter()
            dec.prefill(ids[:n], 0, LLAMA["n_vocab"])
            dt = time.perf_counter() - t1
            prompt[f"level{lvl}"] = {"tokens": n, "s": round(dt, 3), "tokens_per_s": round(n / dt, 1)}
        dec.prompt_mode(1)
    sa.sync()
    t1 = time.perf_counter()
    lg = dec.prefill(ids, 0, LLAMA["n_vocab"])
    dt = time.perf_counter() - t1
    prompt["level1"] = {"tokens": prompt_len, "s": round(dt, 3), "tokens_per_s": round(prompt_len / dt, 1)}
    log(f"prompt of {prompt_len} ids: {prompt}")
    tok = int(np.argmax(lg))
    pos = prompt_len
    warm = dec.generate(tok, pos, W)            # untimed warm-up steps
    tok, pos = int(warm[-1]), pos + W
    sa.sync()
    t1 = time.perf_counter()
    out = dec.generate(tok, pos, K)             # K timed steps, one graph replay per token
    sa.sync()
    dt = time.perf_counter() - t1
    ev_ms = dec.last_ms()
    extra = {"prompt_reading": prompt}
    if not a.gemv_only and not a.no_extra:
        t1 = time.perf_counter()
        extra["batched_decode"] = batched_decode(dec, LLAMA["n_vocab"])
        log(f"batched: {extra['batched_decode']} ({time.perf_counter() - t1:.1f}s)")
    dec.close()
    if not a.no_exact:
        t1 = time.perf_counter()
        extra["exact_decode"] = exact_decode(path, ids, W, K)
        extra["exact_decode"]["vs_fast"] = round(extra["exact_decode"]["tokens_per_s"] / (K / dt), 4)
        log(f"exact decode: {extra['exact_decode']} ({time.perf_counter() - t1:.1f}s)")
    if not a.no_extra:
        t1 = time.perf_counter()
        extra["qwen25_1p5b_decode"] = qwen_decode(work)
        log(f"qwen2.5-1.5b decode: {extra['qwen25_1p5b_decode']} ({time.perf_counter() - t1:.1f}s)")
        t1 = time.perf_counter()
        extra["small_m_gemm"] = small_gemm(work)
        log(f"small-M GEMM (16 rows): {extra['small_m_gemm']} ({time.perf_counter() - t1:.1f}s)")
        t1 = time.perf_counter()
        extra["moe_layer"] = moe_layer(work)
        log(f"moe: {extra['moe_layer']} ({time.perf_counter() - t1:.1f}s)")
        t1 = time.perf_counter()
        extra["width_sweep"] = width_sweep(work)
        log(f"width sweep ({time.perf_counter() - t1:.1f}s): " +
            ", ".join(f"{k} {v['GB/s']}" for k, v in extra["width_sweep"].items()))
        t1 = time.perf_counter()
        extra["ingest"] = ingest_leg()
        log(f"ingest: {extra['ingest']} ({time.perf_counter() - t1:.1f}s)")
    tps = K / dt
    kv_bytes = 2 * LLAMA["n_layer"] * LLAMA["n_head_kv"] * 128 * 2 * (pos + K / 2)
    roof_tps = HBM_PEAK_GBS * 1e9 / wbytes
    roof_tps_kv = HBM_PEAK_GBS * 1e9 / (wbytes + kv_bytes)
    log(f"decode: {K} tokens in {dt * 1e3:.1f} ms wall ({ev_ms:.1f} ms GPU events): {tps:.1f} tok/s; "
        f"roofline {roof_tps:.0f} tok/s weights-only, {roof_tps_kv:.0f} with KV")
    cpu = None
    if not a.no_cpu:
        t1 = time.perf_counter()
        gp = {"q4_8960x1536": os.path.join(work, "cpu_q4_8960x1536.ssf")}
        sa.synth_matrix(gp["q4_8960x1536"], 8960, 1536, nbits=4, seed=1001)
        for nb in (2, 3, 4, 5, 6, 8):
            for rows, cols in ((4096, 14336), (14336, 4096)):
                p = os.path.join(work, f"cpu_q{nb}_{rows}x{cols}.ssf")
                sa.synth_matrix(p, rows, cols, nbits=nb, seed=1004)
                gp[f"q{nb}_{rows}x{cols}"] = p
        cpu = cpu_baseline(path, pos, extra.get("moe_layer", {}).get("path"), gp)
        for p in gp.values():
            os.remove(p)
        log(f"cpu baseline: {cpu} ({time.perf_counter() - t1:.1f}s)")
    if "moe_layer" in extra and extra["moe_layer"].get("path"):
        os.remove(extra["moe_layer"].pop("path"))
    return {
        "metric": "Q4 GEMV HBM GB/s (% of peak); batch-1 decode tokens/s, Llama-3-8B shape",
        "value": round(tps, 2), "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(dt * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8xq4 (int32 dot, fp32 epilogue)", "data": "synthetic",
        "config": {"workload": "Llama-3-8B-shaped decoder, random-init Q4 SSF weights (32 layers, hidden 4096, "
                               "FFN 14336 SwiGLU, 32/8 heads, head_dim 128, vocab 128256, rope theta 5e5), "
                               "fp16 KV cache, batch-1 greedy decode at positions "
                               f"{pos}..{pos + K - 1} of a {N_CTX}-position context",
                   "global_batch": 1, "seq_len": N_CTX, "parallelism": "single GPU"},
        "decode": {"tokens_per_s": round(tps, 2), "gpu_event_ms": round(ev_ms, 3),
                   "weight_bytes_per_token": wbytes, "kv_bytes_per_token_avg": int(kv_bytes),
                   "roofline_tokens_per_s_weights_only": round(roof_tps, 1),
                   "roofline_tokens_per_s_with_kv": round(roof_tps_kv, 1),
                   "frac_of_weights_roofline": round(tps / roof_tps, 4),
                   "frac_of_weights_kv_roofline": round(tps / roof_tps_kv, 4),
                   "effective_GB/s": round((wbytes + kv_bytes) * tps / 1e9, 1),
                   "first_tokens": [int(t) for t in out[:8]]},
        "gemv_q4": gemv,
        **extra,
        "roofline": roof,
        "cpu_baseline": cpu,
    }


if __name__ == "__main__":
    main()
