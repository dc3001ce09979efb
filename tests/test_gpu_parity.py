"""GPU parity: the HIP path through the C ABI against the CPU oracle, same seeded inputs.

Bars: dequantised weights and top-k indices bit-exact;
fp32 outputs within 1e-5 relative RMSE (the reference's metric,
tests/host_oracle.h:143-171); greedy tokens identical.
"""
import json
import os

import numpy as np
import pytest

import kanjoos_amd as K
import oracle as O
from conftest import rel_rmse

pytestmark = pytest.mark.gpu

SEED = 0


def say(msg):
    print(msg, flush=True)


def test_device_caps(device):
    say(f"device {device.name.decode()} arch={device.gcn_arch.decode()} cus={device.cu_count} "
        f"wave={device.wave_size}")
    assert device.wave_size == 64
    assert device.cu_count >= 1


@pytest.mark.parametrize("type_id,n_in,rows", [(K.TYPE_Q4_K, 2048, 64), (K.TYPE_Q4_K, 768, 96),
                                               (K.TYPE_Q6_K, 768, 40), (K.TYPE_Q6_K, 2048, 8)])
def test_dequant_bit_exact(device, type_id, n_in, rows):
    say(f"dequant type={type_id} n_in={n_in} rows={rows}")
    w = O.synth_tensor(O.tensor_key(SEED, 3, "gate", 5), type_id, n_in, rows)
    want = O.dequant(type_id, w, n_in * rows)
    dw = K.DeviceBuffer.from_array(w)
    out = K.DeviceBuffer(4 * n_in * rows)
    K.dequant(type_id, dw, n_in * rows, out)
    got = out.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("type_id,n_in,n_out", [
    (K.TYPE_Q4_K, 2048, 5120), (K.TYPE_Q4_K, 4096, 2048), (K.TYPE_Q4_K, 768, 2048),
    (K.TYPE_Q4_K, 256, 33), (K.TYPE_Q6_K, 768, 2048), (K.TYPE_Q6_K, 2048, 1000),
    (K.TYPE_BF16, 2048, 3000), (K.TYPE_F32, 2048, 128)])
def test_gemv_vs_oracle(device, type_id, n_in, n_out):
    say(f"gemv type={type_id} n_in={n_in} n_out={n_out}")
    w = O.synth_tensor(O.tensor_key(SEED, 1, "q", -1), type_id, n_in, n_out)
    x = O.synth_f32(O.tensor_key(SEED, 1, "input"), n_in)
    want = O.matmul(type_id, w, n_in, n_out, x)[0]
    dw, dx = K.DeviceBuffer.from_array(w), K.DeviceBuffer.from_array(x)
    dy = K.DeviceBuffer(4 * n_out)
    K.gemv(type_id, dw, n_in, n_out, dx, dy)
    got = dy.download(np.float32)
    assert rel_rmse(got, want) <= 1e-5


def test_gemv_fused_norm_and_residual(device):
    n_in, n_out = 2048, 512
    w = O.synth_tensor(O.tensor_key(SEED, 2, "k", -1), K.TYPE_Q4_K, n_in, n_out)
    x = O.synth_f32(O.tensor_key(SEED, 2, "input"), n_in)
    nw = (1.0 + 0.1 * O.synth_f32(O.tensor_key(SEED, 2, "input", 7), n_in)).astype(np.float32)
    r = O.synth_f32(O.tensor_key(SEED, 2, "input", 8), n_out)
    xn = O.rmsnorm(x, nw, 1e-6)
    want = r + O.matmul(K.TYPE_Q4_K, w, n_in, n_out, xn)[0]
    dy = K.DeviceBuffer(4 * n_out)
    K.gemv(K.TYPE_Q4_K, K.DeviceBuffer.from_array(w), n_in, n_out, K.DeviceBuffer.from_array(x), dy,
           norm_w=K.DeviceBuffer.from_array(nw), eps=1e-6, resid=K.DeviceBuffer.from_array(r))
    assert rel_rmse(dy.download(np.float32), want) <= 1e-5


def moe_layer_inputs(n_embd=2048, n_ff=768, n_expert=128, type_down=K.TYPE_Q4_K, layer=0):
    """One MoE layer, one token: x ~ N(0,1), router f32 ~ N(0,0.02), Q4_K experts ~ N(0,0.02)."""
    x = O.synth_f32(O.tensor_key(SEED, layer, "input"), n_embd)
    router = O.synth_tensor(O.tensor_key(SEED, layer, "router"), K.TYPE_F32, n_embd, n_expert)
    gate = np.concatenate([O.synth_tensor(O.tensor_key(SEED, layer, "gate", e), K.TYPE_Q4_K, n_embd, n_ff)
                           for e in range(n_expert)])
    up = np.concatenate([O.synth_tensor(O.tensor_key(SEED, layer, "up", e), K.TYPE_Q4_K, n_embd, n_ff)
                         for e in range(n_expert)])
    down = np.concatenate([O.synth_tensor(O.tensor_key(SEED, layer, "down", e), type_down, n_ff, n_embd)
                           for e in range(n_expert)])
    return x, router, gate, up, down


@pytest.mark.parametrize("type_down", [K.TYPE_Q4_K, K.TYPE_Q6_K])
def test_moe_decode_layer_config1(device, type_down):
    n_embd, n_ff, n_expert, k = 2048, 768, 128, 8
    say(f"moe layer config1 type_down={type_down}")
    x, router, gate, up, down = moe_layer_inputs(type_down=type_down)
    ones = np.ones(n_embd, np.float32)
    hx = O.rmsnorm(x, ones, 1e-6)
    out_w, logits_w, ti_w, tw_w = O.moe(hx, router, gate, up, down, n_embd, n_ff, n_expert, k,
                                       type_down=type_down)
    d = {n: K.DeviceBuffer.from_array(a) for n, a in
         dict(x=x, router=router, gate=gate, up=up, down=down, ones=ones).items()}
    out = K.DeviceBuffer(4 * n_embd)
    logits = K.DeviceBuffer(4 * n_expert)
    ti = K.DeviceBuffer(4 * k)
    tw = K.DeviceBuffer(4 * k)
    K.moe_decode_layer(d["x"], d["router"], d["gate"], d["up"], d["down"], n_embd, n_ff, n_expert, k,
                       out, logits, ti, tw, norm_w=d["ones"], eps=1e-6, type_down=type_down)
    got_ti = ti.download(np.int32)
    assert list(got_ti) == list(ti_w[0]), (got_ti, ti_w[0])
    assert rel_rmse(logits.download(np.float32), logits_w[0]) <= 1e-5
    assert np.allclose(tw.download(np.float32), tw_w[0], rtol=1e-5, atol=1e-7)
    assert rel_rmse(out.download(np.float32), out_w[0]) <= 1e-5


@pytest.fixture(scope="module")
def config1_weights():
    return moe_layer_inputs()


@pytest.fixture(scope="module")
def q6_down_weights():
    return moe_layer_inputs(type_down=K.TYPE_Q6_K)


@pytest.mark.parametrize("m,type_down", [(1, K.TYPE_Q4_K), (7, K.TYPE_Q4_K), (64, K.TYPE_Q4_K),
                                         (300, K.TYPE_Q4_K), (512, K.TYPE_Q4_K), (7, K.TYPE_Q6_K),
                                         (64, K.TYPE_Q6_K), (512, K.TYPE_Q6_K)])
def test_moe_batch_layer(device, config1_weights, q6_down_weights, m, type_down):
    """Config 2 (m = 512) and smaller batches: the batched MoE layer against the
    oracle's Model::moe on the same m rows (top-k bit-exact, out <= 1e-5), with
    Q4_K or Q6_K (d * sc * (q - 32) per 16 weights) expert down."""
    n_embd, n_ff, n_expert, k = 2048, 768, 128, 8
    say(f"moe batch layer m={m} type_down={type_down}")
    w = config1_weights if type_down == K.TYPE_Q4_K else q6_down_weights
    _, router, gate, up, down = w
    rng = np.random.default_rng(100 + m)
    x = rng.standard_normal((m, n_embd)).astype(np.float32)
    resid = rng.standard_normal((m, n_embd)).astype(np.float32)
    ones = np.ones(n_embd, np.float32)
    hx = np.stack([O.rmsnorm(x[t], ones, 1e-6) for t in range(m)])
    out_w, logits_w, ti_w, tw_w = O.moe(hx, router, gate, up, down, n_embd, n_ff, n_expert, k,
                                       type_down=type_down)
    d = {nm: K.DeviceBuffer.from_array(a) for nm, a in
         dict(x=x, resid=resid, router=router, gate=gate, up=up, down=down, ones=ones).items()}
    out = K.DeviceBuffer(4 * m * n_embd)
    logits = K.DeviceBuffer(4 * m * n_expert)
    ti = K.DeviceBuffer(4 * m * k)
    tw = K.DeviceBuffer(4 * m * k)
    K.moe_batch_layer(d["x"], d["router"], d["gate"], d["up"], d["down"], m, n_embd, n_ff, n_expert,
                      k, out, logits, ti, tw, norm_w=d["ones"], eps=1e-6, resid=d["resid"],
                      type_down=type_down)
    got_ti = ti.download(np.int32).reshape(m, k)
    bad = np.flatnonzero((got_ti != ti_w).any(axis=1))
    assert bad.size == 0, f"top-k differs for tokens {bad[:8]}"
    assert rel_rmse(logits.download(np.float32), logits_w.reshape(-1)) <= 1e-5
    assert np.allclose(tw.download(np.float32).reshape(m, k), tw_w, rtol=1e-5, atol=1e-7)
    got = out.download(np.float32).reshape(m, n_embd) - resid
    worst = max(rel_rmse(got[t], out_w[t]) for t in range(m))
    say(f"  worst per-token rel-RMSE {worst:.3g}")
    assert worst <= 1e-5


@pytest.mark.parametrize("m,seed", [(64, 764), (512, 1213)])
def test_moe_batch_layer_skewed(device, config1_weights, m, seed):
    """Routing concentrated on a few experts: every token is one shared
    direction plus small noise, so most experts get no pair and a handful get
    about m pairs each (many 32-pair or 8-pair work items per expert, the
    grouped kernels' XCD-ordered items of one expert side by side).  Same bar
    as test_moe_batch_layer.  With tokens this alike, some seeds give a token
    two top-9 logits within one float32 ulp, whose selection order then
    depends on the summation order of the logit (not a fixed property of
    either side); the seeds here keep every top-9 gap above 1e-5 relative,
    and the test checks that premise."""
    n_embd, n_ff, n_expert, k = 2048, 768, 128, 8
    say(f"moe batch layer skewed m={m}")
    _, router, gate, up, down = config1_weights
    rng = np.random.default_rng(seed)
    base = rng.standard_normal(n_embd).astype(np.float32)
    x = (base[None, :] + 0.05 * rng.standard_normal((m, n_embd))).astype(np.float32)
    resid = rng.standard_normal((m, n_embd)).astype(np.float32)
    ones = np.ones(n_embd, np.float32)
    hx = np.stack([O.rmsnorm(x[t], ones, 1e-6) for t in range(m)])
    out_w, logits_w, ti_w, tw_w = O.moe(hx, router, gate, up, down, n_embd, n_ff, n_expert, k)
    counts = np.bincount(ti_w.reshape(-1), minlength=n_expert)
    say(f"  experts used {np.count_nonzero(counts)}, most pairs on one expert {counts.max()}")
    assert counts.max() >= m // 2  # the routing is skewed as intended
    top9 = -np.sort(-logits_w.reshape(m, n_expert), axis=1)[:, :9]
    gap = (np.abs(np.diff(top9, axis=1)) / np.abs(top9[:, :-1])).min()
    assert gap > 1e-5, f"inputs hold a near-tie in the top-9 logits ({gap:.3g})"
    d = {nm: K.DeviceBuffer.from_array(a) for nm, a in
         dict(x=x, resid=resid, router=router, gate=gate, up=up, down=down, ones=ones).items()}
    out = K.DeviceBuffer(4 * m * n_embd)
    logits = K.DeviceBuffer(4 * m * n_expert)
    ti = K.DeviceBuffer(4 * m * k)
    tw = K.DeviceBuffer(4 * m * k)
    K.moe_batch_layer(d["x"], d["router"], d["gate"], d["up"], d["down"], m, n_embd, n_ff, n_expert,
                      k, out, logits, ti, tw, norm_w=d["ones"], eps=1e-6, resid=d["resid"])
    got_ti = ti.download(np.int32).reshape(m, k)
    bad = np.flatnonzero((got_ti != ti_w).any(axis=1))
    assert bad.size == 0, f"top-k differs for tokens {bad[:8]}"
    assert np.allclose(tw.download(np.float32).reshape(m, k), tw_w, rtol=1e-5, atol=1e-7)
    got = out.download(np.float32).reshape(m, n_embd) - resid
    worst = max(rel_rmse(got[t], out_w[t]) for t in range(m))
    say(f"  worst per-token rel-RMSE {worst:.3g}")
    assert worst <= 1e-5


def small_config(**kw):
    base = dict(n_layer=3, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=256,
                n_expert=16, n_expert_used=4, n_vocab=4096, n_ctx=160)
    base.update(kw)
    return base


def test_model_synth_matches_host_generator(device):
    cfg = small_config()
    m = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    img_gpu = m.download_image()
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    img_cpu = om.image()  # a view into om's memory: om must stay alive
    assert img_gpu.size == img_cpu.size
    bad = np.flatnonzero(img_gpu != img_cpu)
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"


def step_parity(om, gm, tokens, n_layer, tol=1e-5):
    """One decode step per token on both sides.  The oracle adopts the GPU's f16
    value of each new KV element after checking it is the rounding of an f32
    value within 1e-5 of the oracle's own (an f32 difference in the last bits can
    flip an f16 rounding decision, and the flip then propagates at ~1e-5); so the
    per-layer comparison measures every other operation of the step."""
    worst = 0.0
    for t in tokens:
        lg = gm.forward([t])
        kg, vg = gm.kv_download()
        om.set_kv_source(kg, vg)
        lw = om.forward([t])
        st = om.kv_stats()
        assert st["max_mid_dist"] <= 1e-5, st
        for il in range(n_layer):
            e = rel_rmse(gm.hidden(il), om.hidden(il))
            worst = max(worst, e)
            assert e <= tol, (t, il, e)
            assert list(gm.topk(il)[0]) == list(om.topk(il)[0]), (t, il)
        assert rel_rmse(lg, lw) <= tol
    om.set_kv_source(None, None)
    return worst, lg, lw


@pytest.mark.parametrize("cfgkw", [dict(), dict(type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K),
                                   # 64 experts top-6 over 1024-wide rows: the folded router's
                                   # rows and the selection at another shape
                                   dict(n_embd=1024, head_dim=128, n_expert=64, n_expert_used=6)])
def test_small_model_step_parity(device, cfgkw):
    cfg = small_config(**cfgkw)
    say(f"small model per-step parity {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    worst, _, _ = step_parity(om, gm, [11, 22, 33, 44, 55, 66, 77, 88], cfg["n_layer"])
    say(f"worst per-layer rel-RMSE {worst:.3g}")


def test_small_model_step_parity_router_unfolded(device, monkeypatch):
    """The same with KNJ_NO_ROUTER_FOLD=1: the router as a launch of its own
    after the attention output (the path for shapes the folded router does
    not take), and the folded model beside it, each against its own oracle
    model step by step (per-layer hidden and logits <= 1e-5, top-k exact).
    The two GPU models are not held to 1e-5 of each other: each keeps its own
    f16 cache, and a last-bit difference of a layer's input (the router's two
    forms round differently) can flip the f16 rounding of a new cache element,
    which moves that layer's output by up to ~1e-4 (measured: 3.5e-5 at one
    step when both start the step from the same cache); the oracle adopts
    each side's f16 values after checking they are roundings of its own."""
    cfg = small_config()
    say(f"small model per-step parity, router unfolded {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    of = O.OracleModel(O.make_config(**cfg), seed=SEED)
    monkeypatch.setenv("KNJ_NO_ROUTER_FOLD", "1")
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    monkeypatch.delenv("KNJ_NO_ROUTER_FOLD")
    gf = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    toks = [11, 22, 33, 44, 55, 66, 77, 88]
    try:
        worst, lg, _ = step_parity(om, gm, toks, cfg["n_layer"])
        worst_f, lf, _ = step_parity(of, gf, toks, cfg["n_layer"])
        say(f"unfolded: worst per-layer rel-RMSE {worst:.3g}; folded {worst_f:.3g}; folded vs "
            f"unfolded logits after {len(toks)} steps {rel_rmse(lf, lg):.3g}")
    finally:
        gm.close()
        gf.close()
        om.close()
        of.close()


@pytest.mark.parametrize("cfgkw", [dict(), dict(type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K)])
def test_small_model_greedy_parity(device, cfgkw):
    """Free-running greedy decode: each side keeps its own f16 KV cache."""
    cfg = small_config(**cfgkw)
    say(f"small model greedy {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    prompt = [11, 22, 33, 44, 55]
    lw = om.forward(prompt)
    lg = gm.forward(prompt)
    assert int(np.argmax(lg)) == int(np.argmax(lw))
    want = om.greedy([int(np.argmax(lw))], 64)
    got = gm.decode_greedy(int(np.argmax(lg)), 64)
    assert list(got) == list(want)


@pytest.mark.parametrize("n_embd", [2560, 3072])
def test_bf16_head_odd_width_greedy(device, n_embd):
    """A bf16 LM head whose input width has no instantiated fast kernel (2560 and
    3072 = 5 and 6 x 512) runs the general bf16 GEMV; the step's argmax must
    read every one of its per-workgroup keys: per-step parity and free-running
    greedy tokens against the oracle."""
    cfg = small_config(n_layer=2, n_embd=n_embd, n_vocab=6000)
    say(f"bf16 head width {n_embd} {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    step_parity(om, gm, [3, 9], cfg["n_layer"])
    gm.reset()
    om.reset()
    prompt = [5, 6, 7]
    lw = om.forward(prompt)
    lg = gm.forward(prompt)
    assert int(np.argmax(lg)) == int(np.argmax(lw))
    want = om.greedy([int(np.argmax(lw))], 24)
    got = gm.decode_greedy(int(np.argmax(lg)), 24)
    assert list(got) == list(want)
    gm.close()
    om.close()


def prefill_parity(om, gm, prompt, n_layer, tol=1e-5):
    """One forward call over a prompt on both sides (the GPU's prompt pass, the
    oracle's batched Model::forward).  As in step_parity the oracle adopts the
    GPU's f16 cache values after checking each is the rounding of an f32 value
    within 1e-5 of its own, so a flipped rounding does not propagate into
    the comparison of the last row's per-layer residuals, top-k and logits."""
    lg = gm.forward(prompt)
    kg, vg = gm.kv_download()
    om.set_kv_source(kg, vg)
    lw = om.forward(prompt)
    st = om.kv_stats()
    om.set_kv_source(None, None)
    assert st["adopted"] == 2 * n_layer * gm.cfg.n_head_kv * gm.cfg.head_dim * len(prompt), st
    assert st["max_mid_dist"] <= 1e-5, st
    worst = 0.0
    for il in range(n_layer):
        e = rel_rmse(gm.hidden(il), om.hidden(il))
        worst = max(worst, e)
        assert e <= tol, (il, e)
        assert list(gm.topk(il)[0]) == list(om.topk(il)[0]), il
    assert rel_rmse(lg, lw) <= tol
    assert gm.pos == om.pos
    return worst


PREFILL_SHAPES = {
    "g4_d64": dict(),
    "g8_d128": dict(n_head=32, n_head_kv=4, head_dim=128),
    "g1_d64": dict(n_head=4, n_head_kv=4),
    "g2_d128": dict(n_head=8, n_head_kv=4, head_dim=128),
    "q6k_down": dict(type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K),
}


@pytest.mark.parametrize("shape", list(PREFILL_SHAPES))
def test_prefill_parity(device, shape):
    """A prompt in one call, a second prompt continuing from its cache (rows
    at positions past 0, tiles that start mid-chunk), then decode steps from
    the cache the prompt pass wrote."""
    cfg = small_config(**PREFILL_SHAPES[shape])
    say(f"prefill parity {shape} {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    rng = np.random.default_rng(7)
    p1 = [int(t) for t in rng.integers(0, cfg["n_vocab"], 37)]
    p2 = [int(t) for t in rng.integers(0, cfg["n_vocab"], 21)]
    w1 = prefill_parity(om, gm, p1, cfg["n_layer"])
    w2 = prefill_parity(om, gm, p2, cfg["n_layer"])
    w3, _, _ = step_parity(om, gm, [5, 6, 7], cfg["n_layer"])
    say(f"worst per-layer rel-RMSE: prompt {w1:.3g}, continued {w2:.3g}, steps {w3:.3g}")


def test_prefill_crosses_chunks(device):
    """A 600-token prompt: two chunks of the prompt pass (512 + 88 rows)."""
    cfg = small_config(n_ctx=640)
    say(f"prefill across chunks {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, cfg["n_vocab"], 600)]
    worst = prefill_parity(om, gm, prompt, cfg["n_layer"])
    say(f"worst per-layer rel-RMSE {worst:.3g}")


@pytest.mark.parametrize("shape", ["g4_d64", "g8_d128"])
def test_prefill_split_kv(device, shape):
    """A 512-row prompt pass at positions 520-1031: the attention's KV range
    (17 chunks of 64 slots) is split over two workgroups per tile and merged;
    the second split starts at slot 576, past the positions of the rows at
    520-575, which see none of its slots."""
    cfg = small_config(n_ctx=1100, **PREFILL_SHAPES[shape])
    say(f"prefill split-KV {shape} {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    rng = np.random.default_rng(11)
    p1 = [int(t) for t in rng.integers(0, cfg["n_vocab"], 520)]
    p2 = [int(t) for t in rng.integers(0, cfg["n_vocab"], 512)]
    w1 = prefill_parity(om, gm, p1, cfg["n_layer"])
    w2 = prefill_parity(om, gm, p2, cfg["n_layer"])
    say(f"worst per-layer rel-RMSE: {w1:.3g}, split {w2:.3g}")


def test_prefill_edges(device):
    """A 513-token prompt (a 512-row chunk, then a chunk of one row) against the
    oracle; a prompt that fills the context exactly, after which one more
    token is refused as the reference refuses it (model.cpp:514-517)."""
    cfg = small_config(n_ctx=520)
    say(f"prefill edges {cfg}")
    om = O.OracleModel(O.make_config(**cfg), seed=SEED)
    gm = K.Model.from_image(K.qwen3_30b_a3b(**cfg), om.image())
    prompt = [int(t) for t in np.random.default_rng(13).integers(0, cfg["n_vocab"], 513)]
    worst = prefill_parity(om, gm, prompt, cfg["n_layer"])
    say(f"worst per-layer rel-RMSE {worst:.3g}")
    gm.reset()
    gm.forward([1] * cfg["n_ctx"])
    assert gm.pos == cfg["n_ctx"]
    with pytest.raises(K.KnjError, match="context exhausted"):
        gm.forward([2])


def test_prompt_steps_switch(device):
    """KNJ_PROMPT_STEPS=1 feeds a prompt one decode step per token; the prompt
    pass and the steps agree as the reference's batched and single-token
    forwards do (~1e-4: their products round differently)."""
    cfg = small_config()
    prompt = [int(t) for t in np.random.default_rng(21).integers(0, cfg["n_vocab"], 40)]
    a = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    b = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    try:
        la = a.forward(prompt)
        os.environ["KNJ_PROMPT_STEPS"] = "1"
        try:
            lb = b.forward(prompt)
        finally:
            del os.environ["KNJ_PROMPT_STEPS"]
        assert a.pos == b.pos == len(prompt)
        assert not np.array_equal(la, lb)  # the two paths did run
        assert rel_rmse(la, lb) < 3e-4
        for il in range(cfg["n_layer"]):
            assert rel_rmse(a.hidden(il), b.hidden(il)) < 3e-4
    finally:
        a.close()
        b.close()


def test_prefill_errors(device):
    cfg = small_config()
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    with pytest.raises(K.KnjError, match="context exhausted"):
        gm.forward([1] * (cfg["n_ctx"] + 1))
    with pytest.raises(K.KnjError, match="out of range"):
        gm.forward([1, cfg["n_vocab"]])
    assert gm.pos == 0
    gm.forward([1, 2, 3])
    assert gm.pos == 3


def test_cpp_driver_runs(device):
    """The C++ Model/Backend classes end to end through kanjoos-run (small geometry)."""
    import os
    import subprocess

    exe = os.path.join(os.path.dirname(K.LIB_PATH), "kanjoos-run")
    r = subprocess.run([exe, "--small", "--layers", "2", "--ctx", "64", "--prompt", "8",
                        "--n-predict", "16"], capture_output=True, text=True, timeout=60)
    say(r.stdout + r.stderr)
    assert r.returncode == 0
    toks = r.stdout.strip().splitlines()[-1].split()
    assert toks[0] == "tokens:" and len(toks) == 17


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_config1_against_golden(device):
    """One MoE layer, one token, on the GPU against the committed oracle fixture."""
    want = json.load(open(os.path.join(GOLDEN, "config1.json")))
    n_embd, n_ff, n_expert, k = 2048, 768, 128, 8
    x, router, gate, up, down = moe_layer_inputs()
    d = {n: K.DeviceBuffer.from_array(a) for n, a in
         dict(x=x, router=router, gate=gate, up=up, down=down, ones=np.ones(n_embd, np.float32)).items()}
    out, logits = K.DeviceBuffer(4 * n_embd), K.DeviceBuffer(4 * n_expert)
    ti, tw = K.DeviceBuffer(4 * k), K.DeviceBuffer(4 * k)
    K.moe_decode_layer(d["x"], d["router"], d["gate"], d["up"], d["down"], n_embd, n_ff, n_expert, k,
                       out, logits, ti, tw, norm_w=d["ones"], eps=1e-6)
    assert list(ti.download(np.int32)) == want["topk_idx"]
    assert rel_rmse(out.download(np.float32), want["out"]) <= 1e-5


def full_config(**kw):
    return dict(n_ctx=160, **kw)


@pytest.fixture(scope="module")
def full_pair(device):
    """The 48-layer Qwen3-30B-A3B-shaped model on the GPU (seed 0) and the CPU
    oracle over the same (downloaded) weight image."""
    say("full model: generating 18 GB of weights on the GPU")
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**full_config()), seed=SEED)
    img = gm.download_image()
    om = O.OracleModel(O.make_config(**full_config()), seed=SEED, image=img, threads=16)
    yield gm, om, img
    gm.close()
    om.close()


def test_full_model_step_parity(full_pair):
    """Per-layer hidden states (all 48 layers) and top-8 choices on the full model."""
    gm, om, _ = full_pair
    gm.reset()
    om.reset()
    worst, lg, lw = step_parity(om, gm, [1, 2, 3], 48)
    say(f"full model: worst per-layer rel-RMSE {worst:.3g}")


def test_full_model_greedy_golden(device):
    """64 greedy tokens of the full model against the oracle's committed run
    (tests/golden/full_greedy.json, 7 distinct tokens, smallest top-1/top-2
    margin 3.0e-3): identical tokens, and at every step the logits of the
    oracle's 16 largest entries within 1e-2 of the largest logit.  Each side
    keeps its own f16 cache here (nothing is adopted), so the two caches differ
    by f16 rounding flips of single elements, and a flipped key element moves a
    sharp attention score enough to move the logits: measured 1.2e-4 after the
    12-token prompt, 1-2e-4 at most steps, up to 5e-3 at a few.  The 1e-5 bar
    on logits and on every layer is held where the oracle adopts the GPU's
    cache values (test_full_model_step_parity, tests/test_gpu_full_configs.py);
    this test pins the free-running token sequence."""
    path = os.path.join(GOLDEN, "full_greedy.json")
    want = json.load(open(path))
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**full_config()), seed=want["seed"])
    try:
        lg = gm.forward(want["prompt"])
        worst = []
        for step, tok in enumerate(want["tokens"]):
            ids = np.asarray(want["top16_ids"][step])
            ref = np.asarray(want["top16_logits"][step], dtype=np.float64)
            scale = float(np.max(np.abs(ref)))
            err = float(np.max(np.abs(lg[ids].astype(np.float64) - ref))) / scale
            worst.append(err)
            assert int(np.argmax(lg)) == tok, (step, int(np.argmax(lg)), tok)
            assert err <= 1e-2, (step, err)
            if step + 1 < len(want["tokens"]):
                lg = gm.forward([tok])
        say(f"golden: {len(want['tokens'])} tokens ({want['distinct_tokens']} distinct, min margin "
            f"{want['min_margin']:.3g}); logits vs oracle: step 0 {worst[0]:.2e}, max {max(worst):.2e}; all {[round(w * 1e6, 1) for w in worst]}")
    finally:
        gm.close()


def _attn_ref(q, k, v, qn, kn, eps, base, pos, n_head, n_kv, D, kc, vc):
    """float64 restatement of the attention block (model.cpp:560-617): per-head
    RMSNorm, NEOX RoPE, softmax(q.k/sqrt(D)) over slots 0..pos, sum a*v.  The
    rotation angle is formed in float32 as the reference's table is
    (model.cpp:227-230): at base 1e6 a float64 angle differs from it by up to
    pos * 6e-8 rad, far above the tolerance."""
    half = D // 2
    f = np.float32
    # powf of exact exponents: the float64 power rounded once to float32 (numpy's
    # own float32 power may differ from it by a few ulp)
    inv = (float(f(base)) ** (-2.0 * np.arange(half) / D)).astype(f)
    th = (f(pos) * inv).astype(np.float64)
    c, s = np.cos(th), np.sin(th)

    def norm_rope(x, w):
        x = x.astype(np.float64)
        x = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w
        x0, x1 = x[..., :half], x[..., half:]
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], -1)

    qr = norm_rope(q.reshape(n_head, D), qn)
    kr = norm_rope(k.reshape(n_kv, D), kn)
    G = n_head // n_kv
    out = np.zeros((n_head, D))
    for h in range(n_head):
        g = h // G
        K_ = kc[g, :pos + 1].astype(np.float64)
        V_ = vc[g, :pos + 1].astype(np.float64)
        sc = K_ @ qr[h] / np.sqrt(D)
        a = np.exp(sc - sc.max())
        out[h] = (a / a.sum()) @ V_
    return out, kr


@pytest.mark.parametrize("n_head,n_kv,D,pos,n_ctx", [
    (nh, nkv, d, p, 200) for (nh, nkv, d) in [(32, 4, 128), (16, 2, 64), (12, 4, 128), (8, 8, 64)]
    for p in [0, 63, 64, 130, 199]] + [(32, 4, 128, 20000, 32768), (32, 4, 128, 32767, 32768)] +
    # three 64-slot chunks per workgroup (two in flight), with splits past the
    # position and one holding it part-way; five chunks per workgroup
    [(32, 4, 128, 39999, 40000), (32, 4, 128, 160, 40000), (32, 4, 128, 30100, 40000),
     (16, 2, 64, 39000, 40000), (32, 4, 128, 69999, 70000)])
def test_attention_step(device, n_head, n_kv, D, pos, n_ctx):
    """knj_attention_step against a float64 reference: cache append and output
    (the last two cases are config 5's 32K context)."""
    say(f"attention n_head={n_head} n_kv={n_kv} D={D} pos={pos} n_ctx={n_ctx}")
    eps, base = 1e-6, 1e6
    rng = np.random.default_rng(1000 * pos + D + n_head)
    q = rng.standard_normal(n_head * D).astype(np.float32)
    k = rng.standard_normal(n_kv * D).astype(np.float32)
    v = rng.standard_normal(n_kv * D).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kc = (rng.standard_normal((n_kv, n_ctx, D)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((n_kv, n_ctx, D)).astype(np.float16)
    bufs = [K.DeviceBuffer.from_array(a) for a in (q, k, v, qn, kn)]
    dkc, dvc = K.DeviceBuffer.from_array(kc.view(np.uint16)), K.DeviceBuffer.from_array(vc.view(np.uint16))
    dout = K.DeviceBuffer(4 * n_head * D)
    K.attention_step(*bufs, eps, base, pos, n_head, n_kv, D, n_ctx, dkc, dvc, dout)
    got_kc = dkc.download(np.uint16).view(np.float16).reshape(n_kv, n_ctx, D)
    got_vc = dvc.download(np.uint16).view(np.float16).reshape(n_kv, n_ctx, D)
    out = dout.download(np.float32).reshape(n_head, D)
    # appended slot: v rounded to f16; k normalised + rotated, within one f16 ulp
    want_kc, want_vc = kc.copy(), vc.copy()
    want_vc[:, pos] = v.reshape(n_kv, D).astype(np.float16)
    _, kr = _attn_ref(q, k, v, qn, kn, eps, base, pos, n_head, n_kv, D, want_kc, want_vc)
    assert np.array_equal(got_vc.view(np.uint16), want_vc.view(np.uint16))
    kdiff = np.abs(got_kc[:, pos].astype(np.float64) - kr)
    assert np.all(kdiff <= np.spacing(np.abs(kr).astype(np.float16)).astype(np.float64) * 0.5 + 1e-6)
    others = np.ones(n_ctx, bool)
    others[pos] = False
    assert np.array_equal(got_kc[:, others].view(np.uint16), kc[:, others].view(np.uint16))
    # output against the reference over the cache as the device wrote it
    ref_out, _ = _attn_ref(q, k, v, qn, kn, eps, base, pos, n_head, n_kv, D, got_kc, got_vc)
    assert rel_rmse(out, ref_out) <= 1e-5


@pytest.mark.parametrize("cfgkw", [dict(), dict(type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K)])
def test_batch_decode_parity(device, cfgkw):
    """Config 4's batched step on a small model: three sequences with different
    prompts stepped together; every step, every sequence against its own oracle
    model (per-layer hidden <= 1e-5, top-k exact, logits <= 1e-5), with the same
    f16 KV adoption as the single-sequence parity test; bf16 or Q6_K head."""
    cfg = small_config(**cfgkw)
    n_ctx = cfg["n_ctx"]
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    img = gm.download_image()
    B = 3
    batch = K.Batch(gm, B, n_ctx)
    oms = [O.OracleModel(O.make_config(**cfg), seed=SEED, image=img) for _ in range(B)]
    prompts = np.array([[1, 2, 3, 4], [7, 5, 3, 1], [100, 200, 300, 400]], dtype=np.int32)
    toks = prompts
    for step in range(prompts.shape[1] + 3):
        col = toks[:, step] if step < prompts.shape[1] else nxt
        lg = batch.forward(col)
        for s_ in range(B):
            kg, vg = batch.kv_download(s_)
            oms[s_].set_kv_source(kg, vg)
            lw = oms[s_].forward([int(col[s_])])
            st = oms[s_].kv_stats()
            assert st["max_mid_dist"] <= 1e-5, (step, s_, st)
            for il in range(cfg["n_layer"]):
                e = rel_rmse(batch.hidden(il, s_), oms[s_].hidden(il))
                assert e <= 1e-5, (step, s_, il, e)
                assert list(batch.topk(il, s_)[0]) == list(oms[s_].topk(il)[0]), (step, s_, il)
            assert rel_rmse(lg[s_], lw) <= 1e-5, (step, s_)
        nxt = lg.argmax(axis=1).astype(np.int32)
    say(f"batched step parity over {B} sequences, {prompts.shape[1] + 3} steps")
    for om in oms:
        om.close()
    batch.close()
    gm.close()


@pytest.mark.parametrize("cfgkw", [dict(), dict(type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K)])
def test_batch_greedy_matches_single(device, cfgkw):
    """The batched greedy loop and the single-sequence loop give the same tokens
    for every sequence (small model, 24 steps)."""
    cfg = small_config(**cfgkw)
    gm = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    B, steps = 4, 24
    prompts = np.array([[1, 2, 3], [9, 8, 7], [11, 12, 13], [3, 2, 1]], dtype=np.int32)
    batch = K.Batch(gm, B, cfg["n_ctx"])
    for j in range(prompts.shape[1]):
        lg = batch.forward(prompts[:, j])
    first = lg.argmax(axis=1).astype(np.int32)
    got = batch.decode_greedy(first, steps - 1)
    batch.close()
    for s_ in range(B):
        gm.reset()
        f = int(np.argmax(gm.forward(prompts[s_])))
        want = [f] + list(gm.decode_greedy(f, steps - 1))
        have = [int(first[s_])] + [int(t) for t in got[:, s_]]
        assert have == want, (s_, have, want)
    gm.close()


def test_profile_spans(device):
    """knj_model_profile: the same greedy tokens as the graph replay, one span
    per kernel launch, every layer's ops named, spans in stream order without
    overlap, and the span total inside the wall time of the step."""
    cfg = small_config()
    say(f"profile spans {cfg}")
    a = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    b = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    try:
        a.forward([3, 4])
        b.forward([3, 4])
        want = a.decode_greedy(7, 6)
        got, spans, dropped = b.profile(7, 6)
        assert list(got) == list(want)
        assert dropped == 0
        per_step = len(spans) // 6
        assert per_step * 6 == len(spans)
        step0 = spans[:per_step]
        assert step0[0][0] == "embed" and step0[-1][0] == "sample" and step0[-2][0] == "head"
        for il in range(cfg["n_layer"]):
            names = {s[0] for s in step0 if s[1] == il}
            # the router runs in the attention-output launch where the shape allows
            assert names in ({"qkv", "attention", "attn-o", "moe-router", "moe-gate+up+act",
                              "moe-down+scatter"},
                             {"qkv", "attention", "attn-o+moe-router", "moe-gate+up+act",
                              "moe-down+scatter"}), (il, names)
        for s0, s1 in zip(spans, spans[1:]):
            assert s0[3] <= s0[4] <= s1[3] + 1000, (s0, s1)  # 1 us of event rounding
        busy = sum(s[4] - s[3] for s in spans)
        assert 0 < busy <= spans[-1][4] - spans[0][3] + 1000 * len(spans)
        gate = [s[4] - s[3] for s in spans if s[0] == "moe-gate+up+act"]
        assert all(0 < d < 1_000_000 for d in gate)
        h2d, d2h = b.transfer_bytes()
        assert d2h >= 4 * 6 and h2d > 0  # synthetic weights are generated on the device
        assert 0 < K.device_floor(64) < 50_000
    finally:
        a.close()
        b.close()


def test_cpp_driver_profiling(device, tmp_path):
    """kanjoos-run --profiling prints the device-domain table and writes the
    profile files; the tokens are the ones of the run without it."""
    import subprocess

    exe = os.path.join(os.path.dirname(K.LIB_PATH), "kanjoos-run")
    base = [exe, "--small", "--layers", "2", "--ctx", "64", "--prompt", "8", "--n-predict", "16"]
    plain = subprocess.run(base, capture_output=True, text=True, timeout=60)
    prof = subprocess.run(base + ["--profiling", "--profile-warmup", "4", "--profile-dir",
                                  str(tmp_path)], capture_output=True, text=True, timeout=60)
    say(prof.stdout + prof.stderr)
    assert plain.returncode == 0 and prof.returncode == 0
    assert plain.stdout.strip().splitlines()[-1] == prof.stdout.strip().splitlines()[-1]
    assert "clock domain: device" in prof.stdout and "moe-gate+up+act" in prof.stdout
    assert "0 dropped" in prof.stdout
    data = json.load(open(tmp_path / "profile.json"))
    assert data["device_backend"] and data["steps_kept"] == 12 and data["steps_discarded"] == 4
    comps = {c["component"]: c for c in data["components"]}
    assert comps["qkv"]["dev_ns"] > 0 and comps["decode"]["host_ns"] > 0
    assert data["residency"]["vram_pct"] == 100.0 and data["transfer"]["h2d_bytes"] > 0


@pytest.mark.parametrize("case", ["all_equal", "equal_rows", "two_groups"])
def test_moe_routing_ties(device, config1_weights, case):
    """Routing on the device when probabilities tie exactly: equal
    probabilities keep the lower expert first (Model::moe's strict > over
    ascending experts), here against the oracle, which is pinned to that rule
    on the CPU.  The candidate filter of the device top-k sees every group
    maximum equal in the first case and a threshold shared by many experts in
    the others."""
    n_embd, n_ff, n_expert, k = 2048, 768, 128, 8
    x, router, gate, up, down = config1_weights
    r0 = np.frombuffer(np.ascontiguousarray(router).tobytes(), np.float32).reshape(n_expert, n_embd)
    ones = np.ones(n_embd, np.float32)
    hx = O.rmsnorm(x, ones, 1e-6)
    # rows along the normalised input give the largest logits (about 2 and 1)
    big = (hx * np.float32(0.001)).astype(np.float32)
    r = r0 * np.float32(0.01)
    if case == "all_equal":
        r[:] = 0.0
    elif case == "equal_rows":  # five equal leaders, then the ordinary rows
        for e in (100, 37, 64, 5, 120):
            r[e] = big
    else:  # five equal leaders and six equal runners-up straddling eighth place
        for e in (9, 17, 33, 70, 101):
            r[e] = big
        for e in (2, 50, 90, 127, 11, 60):
            r[e] = big * np.float32(0.5)
    r = np.ascontiguousarray(r).view(router.dtype).reshape(router.shape)
    _, _, ti_w, tw_w = O.moe(hx, r, gate, up, down, n_embd, n_ff, n_expert, k)
    d = {n: K.DeviceBuffer.from_array(a) for n, a in
         dict(x=x, router=r, gate=gate, up=up, down=down, ones=ones).items()}
    out = K.DeviceBuffer(4 * n_embd)
    logits = K.DeviceBuffer(4 * n_expert)
    ti = K.DeviceBuffer(4 * k)
    tw = K.DeviceBuffer(4 * k)
    K.moe_decode_layer(d["x"], d["router"], d["gate"], d["up"], d["down"], n_embd, n_ff, n_expert, k,
                       out, logits, ti, tw, norm_w=d["ones"], eps=1e-6)
    got = list(ti.download(np.int32))
    say(f"{case}: device {got} oracle {list(ti_w[0])}")
    assert got == list(ti_w[0])
    want = {"all_equal": list(range(8)), "equal_rows": [5, 37, 64, 100, 120],
            "two_groups": [9, 17, 33, 70, 101, 2, 11, 50]}[case]
    assert got[:len(want)] == want
    assert np.allclose(tw.download(np.float32), tw_w[0], rtol=1e-6, atol=0)


def test_runs_are_bit_identical(device, config1_weights):
    """Fixed reduction order everywhere (no float atomics): the same inputs give
    the same bits on every run -- a prompt pass with split-KV attention, decode
    steps, and the batched MoE layer, each run twice."""
    cfg = small_config(n_ctx=1100)
    a = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    b = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=SEED)
    try:
        prompt = [int(t) for t in np.random.default_rng(5).integers(0, cfg["n_vocab"], 1030)]
        la, lb = a.forward(prompt), b.forward(prompt)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        for il in range(cfg["n_layer"]):
            assert np.array_equal(a.hidden(il).view(np.uint32), b.hidden(il).view(np.uint32))
        ta, tb = a.decode_greedy(int(np.argmax(la)), 8), b.decode_greedy(int(np.argmax(lb)), 8)
        assert list(ta) == list(tb)
        ka, kb = a.kv_download(), b.kv_download()
        assert np.array_equal(ka[0], kb[0]) and np.array_equal(ka[1], kb[1])
    finally:
        a.close()
        b.close()
    n_embd, n_ff, n_expert, k = 2048, 768, 128, 8
    _, router, gate, up, down = config1_weights
    # 96 tokens: the few-pair kernels (8-pair items); 512: the 32-pair kernels
    for m in (96, 512):
        x = np.random.default_rng(6).standard_normal((m, n_embd)).astype(np.float32)
        d = {nm: K.DeviceBuffer.from_array(v) for nm, v in
             dict(x=x, router=router, gate=gate, up=up, down=down).items()}
        outs = []
        for _ in range(2):
            out = K.DeviceBuffer(4 * m * n_embd)
            logits = K.DeviceBuffer(4 * m * n_expert)
            ti = K.DeviceBuffer(4 * m * k)
            tw = K.DeviceBuffer(4 * m * k)
            K.moe_batch_layer(d["x"], d["router"], d["gate"], d["up"], d["down"], m, n_embd, n_ff,
                              n_expert, k, out, logits, ti, tw)
            outs.append(out.download(np.float32))
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), m
