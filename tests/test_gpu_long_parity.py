"""GPU parity over long runs at the benchmark configurations' full widths, against the CPU oracle
(a restatement of /root/reference/src/model/model.cpp:512-672).

  free-running greedy  config 3's workload: the 48-layer model, a 4096-token
                       cache written by the GPU prompt pass, then 64 greedy
                       decode steps on each side with each side's own cache
                       (nothing adopted after the start).  Greedy decode is the
                       reference CLI's loop (/root/reference/src/cli/main.cpp:
                       544-568).  Tokens must be identical at every step, and
                       the logits within 1e-4 relative RMSE of the oracle's
                       (measured ~2e-6: at 4096 slots the attention is diffuse,
                       so the f16 rounding flips between the two caches move it
                       little); each step's top-1/top-2 margin and logit
                       difference are printed.  With random-init weights and a
                       4096-id random prompt, greedy decode falls into a cycle
                       of one to three tokens for every one of 40 prompt seeds
                       tried (4096-4135, GPU only); the prompt uses seed 4121,
                       the one whose cycle has three distinct tokens.
  config 5 greedy      the same over config 5's workload: Q6_K expert down and
                       LM head, a 32768-token cache written by the GPU prompt
                       pass, 64 free-running greedy steps (measured: one
                       repeated token, smallest top-1/top-2 margin 5.4% of the
                       largest logit, logits within 4.9e-6 of the oracle's at
                       every step).
  config 4 greedy      32 sequences whose caches the GPU prompt pass wrote
                       (2048 ids each) decode 32 lockstep greedy steps; 4 of
                       them free-running against their own oracle models
                       (measured: each a repeated token, smallest margin 1.1%
                       of the largest logit, logits within 1.9e-6).
  prompt pass          the prompt pass itself at full width (2048 hidden, 32/4
                       heads x 128, 128 experts top-8) against the oracle's
                       batched forward (model.cpp:354-364 matmul with m > 1,
                       every key appended before the causal attention): 2
                       layers over 4096 rows, and 1 layer over 8192 rows so the
                       attention's KV range is split over many workgroups and
                       merged.  The oracle computes its own cache and checks
                       every element the GPU wrote (all rows, all layers) to be
                       the f16 rounding of an f32 value within 1e-5 of its own
                       before using it; the last row's per-layer hidden state
                       (<= 1e-5 relative RMSE), its top-8 (identical) and the
                       logits (<= 1e-5) are compared.
"""
import numpy as np
import pytest

import kanjoos_amd as K
import oracle as O
from conftest import progress, rel_rmse

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(1200)]

SEED = 0
THREADS = 16


def margin(lg):
    """top-1 minus top-2 of a logit vector, and the top-1 index."""
    i2 = np.argpartition(lg, -2)[-2:]
    a, b = float(lg[i2[0]]), float(lg[i2[1]])
    return abs(a - b), int(i2[1] if b >= a else i2[0])


def test_config3_free_running_greedy_64(device):
    ctx, steps = 4096, 64
    cfg = dict(n_ctx=ctx + steps + 8)
    progress("free-running greedy: 48-layer model, GPU prompt pass over 4096 random ids")
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    om = None
    try:
        prompt = [int(t) for t in np.random.default_rng(4121).integers(0, 151936, ctx)]
        lg = gm.forward(prompt)
        assert gm.pos == ctx
        img = gm.download_image()
        om = O.OracleModel(O.make_config(**cfg), seed=SEED, image=img, threads=THREADS)
        del img
        k, v = gm.kv_download()
        ok, ov = om.kv()
        ok[...] = k
        ov[...] = v
        del k, v
        om.set_pos(ctx)
        # both sides start from the prompt's greedy token; from here each keeps
        # its own cache
        tok = int(np.argmax(lg))
        toks_g, toks_o, rows = [tok], [tok], []
        tg = to = tok
        for s in range(steps):
            lg = gm.forward([tg])
            lw = om.forward([to])
            tg, to = int(np.argmax(lg)), int(np.argmax(lw))
            mo, _ = margin(lw)
            scale = float(np.max(np.abs(lw)))
            diff = float(np.max(np.abs(lg.astype(np.float64) - lw))) / scale
            rows.append((s, to, mo / scale, diff))
            progress(f"greedy step {s} at pos {gm.pos - 1}: gpu {tg} oracle {to}, oracle margin "
                     f"{mo / scale:.3g} of the largest logit, max |logit diff| {diff:.3g}, "
                     f"rel-RMSE {rel_rmse(lg, lw):.3g}")
            assert tg == to, (s, tg, to, mo / scale, diff)
            assert rel_rmse(lg, lw) <= 1e-4, (s, rel_rmse(lg, lw))
            toks_g.append(tg)
            toks_o.append(to)
        assert toks_g == toks_o
        progress(f"free-running greedy: {steps} steps identical ({len(set(toks_g))} distinct tokens), "
                 f"smallest margin {min(r[2] for r in rows):.3g}, largest logit diff "
                 f"{max(r[3] for r in rows):.3g}")
    finally:
        if om is not None:
            om.close()
        gm.close()


def test_config5_free_running_greedy_64(device):
    """Config 5's workload free-running: the 48-layer model with Q6_K expert
    down and LM head, a 32768-slot cache written by the GPU prompt pass (in
    calls of 4096 ids), then 64 greedy steps on each side with its own cache.
    Tokens must be identical at every step and the logits within 1e-4
    relative RMSE of the oracle's."""
    ctx, steps = 32768, 64
    cfg = dict(n_ctx=ctx + steps + 8, type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K)
    progress("config 5 free-running greedy: 48-layer Q6_K-down/head model, GPU prompt pass over 32768 ids")
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    om = None
    try:
        prompt = np.random.default_rng(32768).integers(0, 151936, ctx).astype(np.int32)
        lg = None
        for c0 in range(0, ctx, 4096):
            lg = gm.forward(prompt[c0:c0 + 4096], want_logits=c0 + 4096 >= ctx)
            progress(f"config 5 free-running greedy: prompt pass at {gm.pos}")
        assert gm.pos == ctx
        img = gm.download_image()
        om = O.OracleModel(O.make_config(**cfg), seed=SEED, image=img, threads=THREADS)
        del img
        k, v = gm.kv_download()
        ok, ov = om.kv()
        ok[...] = k
        ov[...] = v
        del k, v
        om.set_pos(ctx)
        tok = int(np.argmax(lg))
        toks, rows = [tok], []
        tg = to = tok
        for st in range(steps):
            lg = gm.forward([tg])
            lw = om.forward([to])
            tg, to = int(np.argmax(lg)), int(np.argmax(lw))
            mo, _ = margin(lw)
            scale = float(np.max(np.abs(lw)))
            diff = float(np.max(np.abs(lg.astype(np.float64) - lw))) / scale
            rows.append((st, to, mo / scale, diff))
            progress(f"config 5 greedy step {st} at pos {gm.pos - 1}: gpu {tg} oracle {to}, oracle margin "
                     f"{mo / scale:.3g} of the largest logit, max |logit diff| {diff:.3g}, "
                     f"rel-RMSE {rel_rmse(lg, lw):.3g}")
            assert tg == to, (st, tg, to, mo / scale, diff)
            assert rel_rmse(lg, lw) <= 1e-4, (st, rel_rmse(lg, lw))
            toks.append(tg)
        progress(f"config 5 free-running greedy: {steps} steps identical ({len(set(toks))} distinct tokens), "
                 f"smallest margin {min(r[2] for r in rows):.3g}, largest logit diff "
                 f"{max(r[3] for r in rows):.3g}")
    finally:
        if om is not None:
            om.close()
        gm.close()


def test_config4_free_running_greedy_32(device):
    """Config 4's workload free-running: 32 sequences, each cache written by a
    GPU prompt pass over 2048 ids, then 32 lockstep greedy steps of the batch
    (every sequence fed its own argmax); 4 of the sequences decode on their
    own oracle model from the same cache, each side keeping its own cache.
    Tokens must be identical at every step and the logits within 1e-4
    relative RMSE of the oracle's."""
    n_seq, ctx, steps, check = 32, 2048, 32, 4
    cfg = dict(n_ctx=ctx + steps + 8)
    progress("config 4 free-running greedy: 48-layer model, 32 prompt passes of 2048 ids")
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    batch = K.Batch(gm, n_seq, ctx + steps + 8)
    oms = []
    try:
        img = gm.download_image()
        picked = list(range(3, n_seq, n_seq // check))
        rng = np.random.default_rng(20480)
        first = np.zeros(n_seq, np.int32)
        for sq in range(n_seq):
            gm.reset()
            lg = gm.forward([int(t) for t in rng.integers(0, 151936, ctx)])
            first[sq] = int(np.argmax(lg))
            k, v = gm.kv_download()
            batch.kv_upload(sq, k, v)
            if sq in picked:
                om = O.OracleModel(O.make_config(**cfg), seed=SEED, image=img, threads=THREADS)
                ok, ov = om.kv()
                ok[...] = k
                ov[...] = v
                om.set_pos(ctx)
                oms.append(om)
        del img
        batch.set_pos(ctx)
        tg = first.copy()
        to = [int(first[sq]) for sq in picked]
        seqs = [[t] for t in to]
        worst, smallest = 0.0, 1.0
        for st in range(steps):
            lg = batch.forward(tg)
            tg = lg.argmax(axis=1).astype(np.int32)
            for j, sq in enumerate(picked):
                lw = oms[j].forward([to[j]])
                to[j] = int(np.argmax(lw))
                mo, _ = margin(lw)
                e = rel_rmse(lg[sq], lw)
                worst, smallest = max(worst, e), min(smallest, mo / float(np.max(np.abs(lw))))
                assert int(tg[sq]) == to[j], (st, sq, int(tg[sq]), to[j])
                assert e <= 1e-4, (st, sq, e)
                seqs[j].append(to[j])
            progress(f"config 4 greedy step {st}: sequences {picked} tokens {[int(tg[q]) for q in picked]}, "
                     f"worst logits rel-RMSE so far {worst:.3g}")
        progress(f"config 4 free-running greedy: {steps} steps identical on {check} sequences "
                 f"({[len(set(q)) for q in seqs]} distinct tokens), smallest margin {smallest:.3g}, "
                 f"largest logits rel-RMSE {worst:.3g}")
    finally:
        for om in oms:
            om.close()
        batch.close()
        gm.close()


def prompt_pass_vs_oracle(n_layer, n_rows, seed):
    cfg = dict(n_layer=n_layer, n_ctx=n_rows + 8)
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    om = None
    try:
        img = gm.download_image()
        om = O.OracleModel(O.make_config(**cfg), seed=SEED, image=img, threads=THREADS)
        del img
        prompt = [int(t) for t in np.random.default_rng(seed).integers(0, 151936, n_rows)]
        progress(f"prompt pass {n_layer} layers x {n_rows} rows: GPU")
        lg = gm.forward(prompt)
        kg, vg = gm.kv_download()
        om.set_kv_source(kg, vg)
        progress(f"prompt pass {n_layer} layers x {n_rows} rows: oracle's batched forward")
        lw = om.forward(prompt)
        st = om.kv_stats()
        om.set_kv_source(None, None)
        progress(f"prompt pass {n_layer}x{n_rows}: cache check {st}")
        assert st["adopted"] == 2 * n_layer * 4 * 128 * n_rows, st
        # the bar of the full-size configs: RMS distance over all the writes
        # within 1e-5 of the values' RMS, no single element further than 5e-5
        # (elements are O(1); the largest distance sits a few times above the RMS)
        assert st["rel_rms_dist"] <= 1e-5, st
        assert st["max_mid_dist"] <= 5e-5, st
        errs = []
        for il in range(n_layer):
            e = rel_rmse(gm.hidden(il), om.hidden(il))
            errs.append(e)
            assert e <= 1e-5, (il, e)
            assert list(gm.topk(il)[0]) == list(om.topk(il)[0]), il
        el = rel_rmse(lg, lw)
        progress(f"prompt pass {n_layer}x{n_rows}: last row per-layer rel-RMSE {errs}, logits {el:.3g}")
        assert el <= 1e-5, el
        assert int(np.argmax(lg)) == int(np.argmax(lw))
        assert gm.pos == om.pos == n_rows
    finally:
        if om is not None:
            om.close()
        gm.close()


def test_prompt_pass_full_width_4096_rows(device):
    prompt_pass_vs_oracle(2, 4096, 40962)


def test_prompt_pass_full_width_8192_rows(device):
    prompt_pass_vs_oracle(1, 8192, 81921)
