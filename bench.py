#!/usr/bin/env python3
"""Decode benchmark: 48-layer Qwen3-30B-A3B-shaped greedy decode at batch 1 on one MI355X.

Workload: the 48-layer Qwen3-30B-A3B-shaped model (hidden 2048, 32/4 heads x 128
with QK-RMSNorm, RoPE theta 1e6, 128 experts top-8 of width 768, vocab 151936;
Q4_K attention and experts, bf16 embeddings and LM head, synthetic weights
~N(0, 0.02) from seed 0), f16 KV cache filled to --ctx tokens (4096) by one
forward call over random token ids (timed and reported as the prompt pass),
then greedy decode at batch 1.  A step is one decode token:
embed, 48 layers, LM head, argmax -- one replay of the captured step graph.

Prints one JSON line: tokens/s, the roofline of the dominant kernel (the Q4_K
expert gate/up GEMV, timed with HIP events on the stream it runs on), the
whole-token HBM fraction, and the CPU oracle's tokens/s on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import kanjoos_amd as K  # noqa: E402

HBM_PEAK_GBPS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bytes_per_token(cfg: K.ModelConfig, ctx: int) -> dict:
    """Algorithmic HBM bytes of one decode token at context length `ctx`
    (positions attended = ctx): every weight byte the step must read once, the
    KV cache read, the embedding row."""
    H, E, F, k = cfg.n_embd, cfg.n_expert, cfg.n_ff, cfg.n_expert_used
    QD, KVD = cfg.n_head * cfg.head_dim, cfg.n_head_kv * cfg.head_dim
    rb = K.row_bytes
    router = 4 * H * E
    experts = k * (2 * rb(cfg.type_gate_up, H) * F + rb(cfg.type_down, F) * H)
    attn = rb(cfg.type_attn, H) * (QD + 2 * KVD) + rb(cfg.type_attn, QD) * H
    kv = 2 * 2 * cfg.n_head_kv * cfg.head_dim * ctx
    head = rb(cfg.type_head, H) * cfg.n_vocab
    embd = rb(cfg.type_embd, H)
    total = cfg.n_layer * (router + experts + attn + kv) + head + embd
    return dict(total=total, experts_per_layer=experts, router=router, attn=attn,
                kv_per_layer=kv, head=head)


def expert_traffic():
    """HBM bytes per k_expert_gateup launch from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the counters' reading
    for a device copy of known size), or None when it is absent."""
    path = os.path.join(ROOT, "profiles", "k_expert_gateup_traffic.json")
    try:
        with open(path) as f:
            return int(json.load(f)["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def hip_runtime():
    """The HIP runtime's stream, graph and event calls used by the config-1 leg."""
    import ctypes as C

    h = C.CDLL("libamdhip64.so")
    P = C.c_void_p
    for name, argt in [("hipStreamCreate", [C.POINTER(P)]), ("hipStreamDestroy", [P]),
                       ("hipStreamBeginCapture", [P, C.c_int]),
                       ("hipStreamEndCapture", [P, C.POINTER(P)]),
                       ("hipGraphInstantiate", [C.POINTER(P), P, P, P, C.c_size_t]),
                       ("hipGraphLaunch", [P, P]), ("hipStreamSynchronize", [P]),
                       ("hipGraphExecDestroy", [P]), ("hipGraphDestroy", [P]),
                       ("hipEventCreate", [C.POINTER(P)]), ("hipEventRecord", [P, P]),
                       ("hipEventSynchronize", [P]), ("hipEventDestroy", [P]),
                       ("hipEventElapsedTime", [C.POINTER(C.c_float), P, P]),
                       ("hipMemcpy", [P, P, C.c_size_t, C.c_int])]:
        getattr(h, name).argtypes = argt
        getattr(h, name).restype = C.c_int
    return h


def moe_layer_leg(model: K.Model, cfg: K.ModelConfig, reps: int, cpu_threads: int) -> dict:
    """MoE layer leg (config 1): one token through one MoE layer (RMSNorm of
    weight 1, router, softmax/top-8, the 8 routed experts' Q4_K gate/up + SwiGLU
    and down, the weighted sum in ascending expert order, the residual) by the
    C ABI entry point knj_moe_decode_layer_noalloc.  One call per layer of the
    model (its router and 128 experts each: 16.3 GB of experts in rotation, so
    the 256 MB memory-side cache cannot serve a layer's weights again), x ~ N(0,1)
    per layer, captured in one HIP graph; HIP events around `reps` replays on
    the graph's stream.  With cpu_threads > 0, the oracle's Model::moe on layer
    0's weights (copied to the host) is timed beside it on that many threads."""
    import ctypes as C

    H, F, E, k, L = cfg.n_embd, cfg.n_ff, cfg.n_expert, cfg.n_expert_used, cfg.n_layer
    base = model.image_device()
    ptr = lambda off: C.c_void_p(base + off)  # noqa: E731
    rng = np.random.default_rng(1)
    xs = [K.DeviceBuffer.from_array(rng.standard_normal(H).astype(np.float32)) for _ in range(L)]
    ones = K.DeviceBuffer.from_array(np.ones(H, np.float32))
    out = K.DeviceBuffer(4 * H)
    logits = K.DeviceBuffer(4 * E)
    ti = K.DeviceBuffer(4 * k)
    tw = K.DeviceBuffer(4 * k)
    los = [model.layer_offsets(il) for il in range(L)]
    h = hip_runtime()
    P = C.c_void_p
    s, graph, exe, e0, e1 = P(), P(), P(), P(), P()
    assert h.hipStreamCreate(C.byref(s)) == 0
    try:
        def layer(il):
            lo = los[il]
            K.moe_decode_layer_noalloc(xs[il], ptr(lo.router), ptr(lo.gate), ptr(lo.up), ptr(lo.down),
                                       H, F, E, k, out, logits, ti, tw, norm_w=ones, eps=1e-6,
                                       resid=xs[il], stream=s.value)
        for il in range(L):  # eager pass: set-up outside the capture
            layer(il)
        assert h.hipStreamSynchronize(s) == 0
        assert h.hipStreamBeginCapture(s, 2) == 0  # relaxed capture mode
        for il in range(L):
            layer(il)
        assert h.hipStreamEndCapture(s, C.byref(graph)) == 0
        assert h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for _ in range(2):
            assert h.hipGraphLaunch(exe, s) == 0
        assert h.hipEventCreate(C.byref(e0)) == 0 and h.hipEventCreate(C.byref(e1)) == 0
        assert h.hipEventRecord(e0, s) == 0
        for _ in range(reps):
            assert h.hipGraphLaunch(exe, s) == 0
        assert h.hipEventRecord(e1, s) == 0
        assert h.hipEventSynchronize(e1) == 0
        ms = C.c_float()
        assert h.hipEventElapsedTime(C.byref(ms), e0, e1) == 0
    finally:
        for ev in (e0, e1):
            if ev.value:
                h.hipEventDestroy(ev)
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        h.hipStreamSynchronize(s)
        h.hipStreamDestroy(s)
    us = ms.value * 1e3 / (reps * L)
    # bytes per layer-token: router rows, the 8 experts' gate/up/down rows, x in, out
    wbytes = 4 * H * E + k * (2 * K.row_bytes(cfg.type_gate_up, H) * F + K.row_bytes(cfg.type_down, F) * H)
    nbytes = wbytes + 4 * H * 2
    gbps = nbytes / (us * 1e-6) / 1e9
    log(f"config 1: one MoE layer, one token: {us:.2f} us per layer ({gbps:.0f} GB/s, "
        f"{100 * gbps / HBM_PEAK_GBPS:.1f}% of HBM peak)")
    cpu = None
    if cpu_threads > 0:
        import oracle as O  # the CPU baseline only (the checker's C restatement)

        lo = los[0]
        def host(off, n):
            a = np.empty(n, np.uint8)
            assert h.hipMemcpy(a.ctypes.data, base + off, n, 2) == 0  # device to host
            return a
        n_gu = E * F * K.row_bytes(cfg.type_gate_up, H)
        router = host(lo.router, 4 * H * E).view(np.float32)
        gate, up = host(lo.gate, n_gu), host(lo.up, n_gu)
        down = host(lo.down, E * H * K.row_bytes(cfg.type_down, F))
        x0 = xs[0].download(np.float32)
        hx = (x0 / np.sqrt(np.mean(x0.astype(np.float64) ** 2) + 1e-6)).astype(np.float32)
        O.moe(hx, router, gate, up, down, H, F, E, k, threads=cpu_threads)  # warm-up
        best = float("inf")
        for _ in range(10):
            t0 = time.perf_counter()
            O.moe(hx, router, gate, up, down, H, F, E, k, threads=cpu_threads)
            best = min(best, time.perf_counter() - t0)
        cpu = {"us_per_layer": round(best * 1e6, 1), "threads": cpu_threads, "kind": "port",
               "sample": "best of 10 calls of the oracle's Model::moe, one token, layer 0"}
        log(f"config 1 on the CPU oracle ({cpu_threads} threads): {best * 1e6:.0f} us per layer")
    return {"workload": "config 1: one token through one MoE layer (router, softmax/top-8, 8 Q4_K "
                        "experts' gate/up + SwiGLU + down, residual) by knj_moe_decode_layer_noalloc, "
                        f"the model's {L} layers in rotation in one HIP graph",
            "us_per_layer": round(us, 3), "bytes_per_layer": nbytes, "achieved_GBps": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "replays": reps, "cpu": cpu}


def moe_batch_leg(model: K.Model, cfg: K.ModelConfig, m: int, iters: int) -> dict:
    """Batched MoE leg (config 2): one MoE layer (the model's layer 0: router, 128 Q4_K
    experts) over m tokens at once, x ~ N(0,1) with ffn_norm, timed with HIP
    events over `iters` calls of knj_moe_batch_layer on the default stream."""
    import ctypes as C

    H, F, E, k = cfg.n_embd, cfg.n_ff, cfg.n_expert, cfg.n_expert_used
    lo = model.layer_offsets(0)
    base = model.image_device()
    rng = np.random.default_rng(2)
    x = K.DeviceBuffer.from_array(rng.standard_normal((m, H)).astype(np.float32))
    out = K.DeviceBuffer(4 * m * H)
    logits = K.DeviceBuffer(4 * m * E)
    ti = K.DeviceBuffer(4 * m * k)
    tw = K.DeviceBuffer(4 * m * k)
    ptr = lambda off: C.c_void_p(base + off)  # noqa: E731

    def call():
        K.moe_batch_layer(x, ptr(lo.router), ptr(lo.gate), ptr(lo.up), ptr(lo.down), m, H, F, E, k,
                          out, logits, ti, tw, norm_w=ptr(lo.ffn_norm), eps=cfg.rms_eps, resid=x)

    for _ in range(3):
        call()
    K.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        call()
    K.synchronize()
    us = (time.perf_counter() - t0) / iters * 1e6
    # algorithmic work: router + 3 expert GEMMs per (token, expert) pair
    flops = 2.0 * m * H * E + 2.0 * m * k * 3 * H * F
    wbytes = 4 * H * E + E * (2 * K.row_bytes(cfg.type_gate_up, H) * F + K.row_bytes(cfg.type_down, F) * H)
    log(f"config 2: MoE layer over {m} tokens in {us:.1f} us ({m / us * 1e6:.0f} tokens/s, "
        f"{flops / us / 1e6:.1f} TFLOP/s)")
    return {"workload": f"config 2: one MoE layer (128 Q4_K experts, top-8) over {m} tokens at once",
            "us_per_layer": round(us, 2), "tokens_per_s": round(m / us * 1e6, 1),
            "algorithmic_tflops": round(flops / us / 1e6, 2), "weight_bytes": wbytes,
            "weight_GBps": round(wbytes / us / 1e3, 1),
            "note": "expert GEMMs on f16 matrix cores with split (hi + lo) activations, two "
                    "matrix-core steps per algorithmic product"}


def long_ctx_leg(seed: int, ctx: int, steps: int) -> dict:
    """Long-context leg (config 5): the Q4_K_M-style mix (Q6_K expert down and LM head),
    batch 1, f16 KV cache written by the prompt pass over `ctx` random token ids
    (calls of 4096 tokens), then `steps` greedy decode steps timed."""
    cfg = K.qwen3_30b_a3b(n_ctx=ctx + steps + 8, type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K)
    model = K.Model.synthetic(cfg, seed=seed)
    prompt = np.random.default_rng(seed + 32768).integers(0, cfg.n_vocab, size=ctx, dtype=np.int32)
    K.synchronize()
    t0 = time.perf_counter()
    logits = None
    for c0 in range(0, ctx, 4096):
        logits = model.forward(prompt[c0:c0 + 4096], want_logits=c0 + 4096 >= ctx)
    K.synchronize()
    prefill_s = time.perf_counter() - t0
    first = int(np.argmax(logits))
    first = int(model.decode_greedy(first, 2)[-1])  # two warm-up steps
    K.synchronize()
    start = model.pos
    t0 = time.perf_counter()
    model.decode_greedy(first, steps)
    K.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    bpt = bytes_per_token(cfg, start + (steps + 1) // 2)
    model.close()
    log(f"config 5: prompt pass over {ctx} tokens {prefill_s:.2f} s; decode at context {start}: "
        f"{ms:.3f} ms/token, {1e3 / ms:.1f} tok/s")
    return {"workload": f"config 5: 48 layers, Q6_K expert down + LM head, batch 1, f16 KV written "
                        f"by the prompt pass over {ctx} random token ids, decode from context {start}",
            "tokens_per_s": round(1e3 / ms, 2), "ms_per_step": round(ms, 4), "steps": steps,
            "prefill_s": round(prefill_s, 3),
            "bytes_per_token": bpt["total"],
            "token_GBps": round(bpt["total"] / (ms * 1e-3) / 1e9, 1)}


def batch_leg(model: K.Model, seed: int, n_seq: int, ctx: int, steps: int) -> dict:
    """Batched-decode leg (config 4): n_seq concurrent greedy sequences on the same weights,
    each with its own f16 KV cache written by a prompt pass over `ctx` random token
    ids (one prompt per sequence, run on `model` and copied into the batch),
    then `steps` lockstep decode steps timed."""
    batch = K.Batch(model, n_seq, ctx + steps + 8)
    rng = np.random.default_rng(seed + 2048)
    t0 = time.perf_counter()
    first = np.empty(n_seq, dtype=np.int32)
    for sq in range(n_seq):
        model.reset()
        lg = model.forward(rng.integers(0, model.cfg.n_vocab, size=ctx, dtype=np.int32))
        first[sq] = int(np.argmax(lg))
        k, v = model.kv_download()
        n = batch.n_ctx
        batch.kv_upload(sq, k[:, :, :n, :], v[:, :, :n, :])
    batch.set_pos(ctx)
    K.synchronize()
    prefill_s = time.perf_counter() - t0
    first = batch.decode_greedy(first, 2)[-1]  # two warm-up steps
    K.synchronize()
    t0 = time.perf_counter()
    batch.decode_greedy(first, steps)
    K.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    batch.close()
    model.reset()
    log(f"config 4: {n_seq} prompt passes of {ctx} tokens {prefill_s:.2f} s; {n_seq} sequences at "
        f"context {ctx}: {ms:.3f} ms/step, {n_seq * 1e3 / ms:.0f} tokens/s")
    return {"workload": f"config 4: {n_seq} concurrent greedy sequences, f16 KV written by a prompt "
                        f"pass over {ctx} random token ids per sequence, lockstep decode",
            "tokens_per_s": round(n_seq * 1e3 / ms, 1), "ms_per_step": round(ms, 4), "steps": steps,
            "prefill_s": round(prefill_s, 3)}


def calib_probe() -> None:
    """Two kernels whose HBM traffic is known exactly: k_gemv_bf16 over a
    2048 x 65536 bf16 matrix (268,435,456 bytes read once; x and y are 8 KiB and
    256 KiB) and k_dequant of 16,777,216 Q4_K weights (9,437,184 bytes read,
    67,108,864 bytes written).  Then the gate/up launch's bytes without its
    routing: the dense Q4_K GEMV (k_gemv_q4k) over 12,288 rows of 2048 weights
    (14,155,776 bytes: the 8 experts x 2 x 768 rows one gate/up launch reads),
    20 launches over 20 different matrices (283 MB, past the 256 MB
    memory-side cache), for its duration and counters."""
    n_in, n_out = 2048, 65536
    w = K.DeviceBuffer(n_in * n_out * 2)
    w.zero()
    x = K.DeviceBuffer(n_in * 4)
    x.zero()
    y = K.DeviceBuffer(n_out * 4)
    n = 1 << 24
    q = K.DeviceBuffer(n // 256 * 144)
    q.zero()
    out = K.DeviceBuffer(n * 4)
    for _ in range(2):
        K.gemv(K.TYPE_BF16, w, n_in, n_out, x, y)
        K.dequant(K.TYPE_Q4_K, q, n, out)
    K.synchronize()
    log("calibration probe: 2 x (bf16 GEMV 256 MiB read, Q4_K dequant 64 MiB write)")
    del w, q, out
    rows = 12288
    mat = K.row_bytes(K.TYPE_Q4_K, n_in) * rows
    big = K.DeviceBuffer(20 * mat)
    big.zero()
    yq = K.DeviceBuffer(4 * rows)
    for i in range(20):
        K.gemv(K.TYPE_Q4_K, big.ptr + i * mat, n_in, rows, x, yq)
    K.synchronize()
    log(f"dense probe: 20 x Q4_K GEMV over {mat} bytes each (one gate/up launch's bytes)")


def host_cpus() -> dict:
    """Logical CPUs, the CPUs this process may run on, physical cores and the
    CPU model, from os and /proc/cpuinfo."""
    info = {"logical": os.cpu_count() or 1, "affinity": len(os.sched_getaffinity(0)),
            "physical": None, "model": None}
    try:
        cores, phys, core = set(), None, None
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and info["model"] is None:
                    info["model"] = val
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    core = val
                elif not key and phys is not None and core is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
        info["physical"] = len(cores) or None
    except OSError:
        pass
    return info


def cpu_baseline(model: K.Model, cfg: K.ModelConfig, cells: list[tuple[int, int]],
                 share: int) -> dict:
    """The CPU oracle (restating the reference's CPU forward pass, with its
    ThreadPool strategy) on the host cores, continuing from the GPU's weights and
    KV cache at the same position.  One cell per thread count: a fresh oracle
    model (the weight image shared, the cache copied), then `tokens` greedy
    decode tokens timed one by one; the best cell is the headline."""
    import oracle as O  # test infrastructure: only the baseline leg uses it

    cpus = host_cpus()
    log(f"cpu baseline: host {cpus}; downloading {model.image_bytes() / 1e9:.1f} GB weight image")
    image = model.download_image()
    ocfg = O.make_config(**cfg.as_dict())
    kg, vg = model.kv_download()
    pos0 = model.pos
    tok0 = int(model.logits().argmax())
    sweep = []
    for ci, (threads, tokens) in enumerate(cells):
        om = O.OracleModel(ocfg, seed=0, image=image, threads=threads)
        ko, vo = om.kv()
        ko[...] = kg
        vo[...] = vg
        om.set_pos(pos0)
        tok = tok0
        if ci == 0:  # page the weight image in once
            t0 = time.perf_counter()
            logits = om.forward([tok])
            log(f"cpu baseline: warmup token {time.perf_counter() - t0:.2f} s")
            om.set_pos(pos0)
        times = []
        for _ in range(tokens):
            t0 = time.perf_counter()
            logits = om.forward([tok])
            times.append(time.perf_counter() - t0)
            tok = int(np.argmax(logits))
        om.close()
        cell = {"threads": threads, "tokens": tokens, "best_s": round(min(times), 4),
                "mean_s": round(float(np.mean(times)), 4), "tokens_per_s": round(1.0 / min(times), 4)}
        sweep.append(cell)
        log(f"cpu baseline: {threads} threads: {cell}")
    best = max(sweep, key=lambda c: c["tokens_per_s"])
    base1 = next((c for c in sweep if c["threads"] == 1), None)
    for c in sweep:
        if base1:
            c["speedup_vs_1"] = round(c["tokens_per_s"] / base1["tokens_per_s"], 2)
    return {"value": best["tokens_per_s"], "unit": "tokens/s", "cores": best["threads"],
            "kind": "port",
            "sample": (f"greedy decode tokens of the 48-layer model at context {pos0} on "
                       f"oracle/libknj_oracle.so, best token time per cell, cells "
                       f"{[(c['threads'], c['tokens']) for c in sweep]} (threads, tokens); the "
                       f"headline is the best cell ({best['threads']} threads)"),
            "host": {"cpu_model": cpus["model"], "logical_cpus": cpus["logical"],
                     "physical_cores": cpus["physical"], "affinity_cpus": cpus["affinity"],
                     "cpu_share": share,
                     "note": "thread counts stop at the GPU box's CPU share per GPU; "
                             "above it the oracle would compete with other jobs' CPUs"},
            "sweep": sweep}


def sweep_cells(spec: str, share: int) -> list[tuple[int, int]]:
    """'1:3,4:8,16:8' -> [(threads, tokens)], thread counts capped at `share`."""
    cells = []
    for part in spec.split(","):
        t, _, n = part.partition(":")
        th = min(int(t), share)
        if th >= 1 and th not in [c[0] for c in cells]:
            cells.append((th, max(1, int(n or 8))))
    return cells


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096, help="KV prefill length before timing")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--expert-steps", type=int, default=8,
                    help="decode steps whose expert launches are timed one by one with events")
    ap.add_argument("--calib-probe", action="store_true",
                    help="also run two streaming kernels of known traffic (a 256 MiB bf16 GEMV "
                         "read, a 256 MiB f32 dequant write) to scale rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE readings")
    ap.add_argument("--no-moe-layer", dest="moe_layer", action="store_false",
                    help="skip the config-1 leg (one MoE layer, one token)")
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="tokens of the config-2 batched MoE layer leg (0 skips it)")
    ap.add_argument("--batch-seqs", type=int, default=32,
                    help="sequences of the config-4 leg (0 skips it)")
    ap.add_argument("--batch-ctx", type=int, default=2048)
    ap.add_argument("--batch-steps", type=int, default=128)
    ap.add_argument("--long-ctx", type=int, default=32768,
                    help="context of the config-5 leg (0 skips it)")
    ap.add_argument("--long-steps", type=int, default=128)
    ap.add_argument("--cpu-sweep", default="1:8,4:8,16:8",
                    help="CPU baseline cells threads:tokens (thread counts capped at --cpu-share)")
    ap.add_argument("--cpu-share", type=int, default=16,
                    help="host threads the GPU box grants one GPU's job")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build runs the decode path on a single GPU "
              "(expert-parallel sharding across GPUs is a design, not implemented here); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    caps = K.open_device(0)
    log(f"device {caps.name.decode()} {caps.gcn_arch.decode()} {caps.cu_count} CUs")
    n_ctx = args.ctx + args.warmup + args.steps + args.expert_steps + 8
    cfg = K.qwen3_30b_a3b(n_ctx=n_ctx)
    t0 = time.perf_counter()
    model = K.Model.synthetic(cfg, seed=args.seed)
    log(f"synthetic weights on GPU: {model.image_bytes() / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")

    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, cfg.n_vocab, size=args.ctx, dtype=np.int32)
    # the context: one forward call over the prompt (the prompt pass: every
    # weight over 512-row chunks, causal attention), timed on its own
    K.synchronize()
    t0 = time.perf_counter()
    if args.ctx:
        model.forward(prompt, want_logits=False)
    K.synchronize()
    prompt_s = max(time.perf_counter() - t0, 1e-9)
    log(f"prompt pass over {args.ctx} tokens in {prompt_s * 1e3:.1f} ms "
        f"({args.ctx / prompt_s:.0f} tok/s, first call: includes its buffer set-up)")

    first = int(model.logits().argmax())
    if args.warmup:
        warm = model.decode_greedy(first, args.warmup)
        first = int(warm[-1])
    K.synchronize()
    start_pos = model.pos
    t0 = time.perf_counter()
    toks = model.decode_greedy(first, args.steps)
    K.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = 1000.0 * elapsed / args.steps
    tok_s = args.steps / elapsed
    log(f"decode {args.steps} steps from pos {start_pos}: {ms_per_step:.3f} ms/token, {tok_s:.1f} tok/s")

    # whole-token HBM accounting at the mean context of the timed steps
    mean_ctx = start_pos + (args.steps + 1) / 2.0
    bpt = bytes_per_token(cfg, int(round(mean_ctx)))
    token_gbps = bpt["total"] / (ms_per_step * 1e-3) / 1e9

    # dominant kernel: expert gate/up GEMV (and down) inside decode steps that
    # continue the timed run; each launch records HIP start/end events of its own
    # execution on the model stream
    us_gu, us_dn = model.time_experts(args.expert_steps)
    H, F, k = cfg.n_embd, cfg.n_ff, cfg.n_expert_used
    bytes_gu = k * 2 * K.row_bytes(cfg.type_gate_up, H) * F
    bytes_dn = k * K.row_bytes(cfg.type_down, F) * H
    gbps_gu = bytes_gu / (us_gu * 1e-6) / 1e9
    gbps_dn = bytes_dn / (us_dn * 1e-6) / 1e9
    gbps_ex = (bytes_gu + bytes_dn) / ((us_gu + us_dn) * 1e-6) / 1e9
    log(f"expert gate/up {us_gu:.2f} us ({gbps_gu:.0f} GB/s), down {us_dn:.2f} us ({gbps_dn:.0f} GB/s)")
    traffic = expert_traffic()
    if args.calib_probe:
        calib_probe()

    # the CPU baseline continues from this model's state, so it runs before the
    # config-4 leg reuses the model for its prompt passes
    cpu = None
    if not args.no_cpu_baseline:
        share = min(args.cpu_share, len(os.sched_getaffinity(0)))
        cpu = cpu_baseline(model, cfg, sweep_cells(args.cpu_sweep, share), share)

    moe_layer = None
    if args.moe_layer:
        share = 0 if args.no_cpu_baseline else min(args.cpu_share, len(os.sched_getaffinity(0)))
        moe_layer = moe_layer_leg(model, cfg, 20, share)
    moe_batch = moe_batch_leg(model, cfg, args.prefill_tokens, 20) if args.prefill_tokens else None
    batched = None
    if args.batch_seqs and args.batch_ctx + args.batch_steps + 8 <= n_ctx:
        batched = batch_leg(model, args.seed, args.batch_seqs, args.batch_ctx, args.batch_steps)

    result = {
        "metric": "decode tokens/s at batch 1 + achieved HBM GB/s (% of 8 TB/s) on Q4_K expert GEMV",
        "value": round(tok_s, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init weights ~N(0,0.02), random prompt token ids)",
        "config": {
            "workload": "config 3: 48-layer Qwen3-30B-A3B-shaped greedy decode, batch 1, "
                        f"f16 KV prefilled to {args.ctx} tokens, Q4_K attention+experts, bf16 embd/head",
            "batch": 1, "ctx_start": start_pos, "n_layer": cfg.n_layer, "n_expert": cfg.n_expert,
            "top_k": cfg.n_expert_used, "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "k_expert_gateup (Q4_K gate+up GEMV of the 8 routed experts, SwiGLU)",
            "bound": "hbm",
            "achieved": round(gbps_gu, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps_gu / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "bytes_per_launch": bytes_gu,
            "avg_us": round(us_gu, 3),
            "down_kernel": {"bytes_per_launch": bytes_dn, "avg_us": round(us_dn, 3),
                            "achieved": round(gbps_dn, 1)},
            "expert_path_GBps": round(gbps_ex, 1),
        },
        "token_roofline": {
            "bytes_per_token": bpt["total"], "achieved": round(token_gbps, 1), "unit": "GB/s",
            "frac": round(token_gbps / HBM_PEAK_GBPS, 4),
        },
        "cpu_baseline": cpu,
        "prompt_pass": {"tokens": int(args.ctx), "ms": round(prompt_s * 1e3, 2),
                        "tokens_per_s": round(args.ctx / prompt_s, 1)} if args.ctx else None,
        "moe_layer": moe_layer,
        "moe_batch": moe_batch,
        "batched_decode": batched,
    }
    model.close()
    if args.long_ctx:
        result["long_context"] = long_ctx_leg(args.seed, args.long_ctx, args.long_steps)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
