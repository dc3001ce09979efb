"""CPU: the oracle's model-level arithmetic against an independent float64 numpy
forward written from the textbook definitions (RMSNorm, NEOX RoPE, GQA softmax
attention, softmax router with top-k renormalisation, SwiGLU experts), plus the
synthetic-weight generator against a numpy Box-Muller of the same hash stream.

These pin the oracle's composition (which tensor feeds which, residual
placement, the rotation pairing, the expert summation) where no reference
vector exists: a transposed operand, a wrong rotation pair or a dropped
residual moves the result far outside the tolerances below.
"""
import numpy as np
import pytest

import oracle as O
from conftest import rel_rmse
from test_oracle_formats import np_q4k, np_q6k

M64 = (1 << 64) - 1


# ------------------------------------------------------------------ synthetic generator

def np_mix64(z):
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def test_synth_is_box_muller_of_splitmix():
    key = O.tensor_key(3, 1, "input", 2)
    n = 4000
    got = O.synth_f32(key, n).astype(np.float64)
    want = np.empty(n)
    for i in range(n):
        h = np_mix64((key + i * 0x9E3779B97F4A7C15) & M64)
        u1 = (2 * (h >> 41) + 1) * 2.0 ** -24
        u2 = (h & 0xFFFFFF) * 2.0 ** -24
        want[i] = np.sqrt(-2.0 * np.log(u1)) * np.cos(2 * np.pi * u2)
    assert np.max(np.abs(got - want)) < 2e-6


def test_synth_moments_and_determinism():
    key = O.tensor_key(0, 0, "input")
    z = O.synth_f32(key, 1 << 20)
    assert abs(z.mean()) < 5e-3
    assert abs(z.std() - 1.0) < 5e-3
    kurt = np.mean(z.astype(np.float64) ** 4) / np.mean(z.astype(np.float64) ** 2) ** 2
    assert abs(kurt - 3.0) < 0.05
    assert np.array_equal(z, O.synth_f32(key, 1 << 20))
    assert not np.array_equal(z[:100], O.synth_f32(O.tensor_key(1, 0, "input"), 100))


@pytest.mark.parametrize("type_id,limit", [(O.TYPE_Q4_K, 0.55), (O.TYPE_Q6_K, 0.55)])
def test_quantiser_error_bound(type_id, limit):
    """Each weight is within ~half a quantisation step of its source value."""
    key = O.tensor_key(0, 2, "up", 3)
    w = O.synth_tensor(key, type_id, 2048, 8, std=0.02)
    src = O.synth_f32(key, 2048 * 8, std=0.02)
    dq = O.dequant(type_id, w, 2048 * 8)
    err = np.abs(dq - src).reshape(-1, 32 if type_id == O.TYPE_Q4_K else 16)
    srcb = src.reshape(err.shape)
    levels = 15 if type_id == O.TYPE_Q4_K else 31
    step = (srcb.max(1) - np.minimum(srcb.min(1), 0)) / levels if type_id == O.TYPE_Q4_K \
        else np.abs(srcb).max(1) / levels
    # 6-bit scale quantisation widens the step by at most ~1/63 relative, plus the min offset
    assert np.all(err.max(1) <= limit * step * 1.2 + 2e-4)
    assert rel_rmse(dq, src) < (0.08 if type_id == O.TYPE_Q4_K else 0.03)


# ------------------------------------------------------------------ numpy float64 model

TINY = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=256, n_expert=8,
            n_expert_used=2, n_vocab=512, n_ctx=16)


def align(v):
    return (v + 255) & ~255


def np_layout(c):
    """Offsets of include/knj_model.h's weight image, restated."""
    rb = lambda t, n: O.row_bytes(t, n)
    H, D = c["n_embd"], c["head_dim"]
    QD, KVD = c["n_head"] * D, c["n_head_kv"] * D
    F, E, V = c["n_ff"], c["n_expert"], c["n_vocab"]
    p = 0
    off = {"embd": 0}
    p = align(p + rb(c["type_embd"], H) * V)
    layers = []
    for _ in range(c["n_layer"]):
        L = {}
        for name, size in (("attn_norm", 4 * H), ("ffn_norm", 4 * H), ("q_norm", 4 * D),
                           ("k_norm", 4 * D), ("wqkv", rb(c["type_attn"], H) * (QD + 2 * KVD)),
                           ("wo", rb(c["type_attn"], QD) * H), ("router", 4 * H * E),
                           ("gate", rb(c["type_gate_up"], H) * F * E),
                           ("up", rb(c["type_gate_up"], H) * F * E),
                           ("down", rb(c["type_down"], F) * H * E)):
            L[name] = (p, size)
            p = align(p + size)
        layers.append(L)
    off["onorm"] = p
    p = align(p + 4 * H)
    off["head"] = p
    p = align(p + rb(c["type_head"], H) * V)
    return off, layers, p


def np_dq(type_id, blob, rows, n_in):
    if type_id == O.TYPE_Q4_K:
        return np_q4k(blob).reshape(rows, n_in)
    if type_id == O.TYPE_Q6_K:
        return np_q6k(blob).reshape(rows, n_in)
    if type_id == O.TYPE_BF16:
        return (blob.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(rows, n_in)
    return blob.view(np.float32).astype(np.float64).reshape(rows, n_in)


class NpModel:
    def __init__(self, c, image):
        self.c = c
        off, layers, total = np_layout(c)
        assert total == image.size
        H, D = c["n_embd"], c["head_dim"]
        QD, KVD = c["n_head"] * D, c["n_head_kv"] * D
        F, E, V = c["n_ff"], c["n_expert"], c["n_vocab"]
        seg = lambda o, n: image[o:o + n]
        self.embd = np_dq(c["type_embd"], seg(0, O.row_bytes(c["type_embd"], H) * V), V, H)
        self.head = np_dq(c["type_head"], seg(off["head"], O.row_bytes(c["type_head"], H) * V), V, H)
        self.onorm = seg(off["onorm"], 4 * H).view(np.float32).astype(np.float64)
        self.L = []
        for L in layers:
            g = lambda name: seg(*L[name])
            wqkv = np_dq(c["type_attn"], g("wqkv"), QD + 2 * KVD, H)
            sgu = O.row_bytes(c["type_gate_up"], H) * F
            sdn = O.row_bytes(c["type_down"], F) * H
            self.L.append(dict(
                attn_norm=g("attn_norm").view(np.float32).astype(np.float64),
                ffn_norm=g("ffn_norm").view(np.float32).astype(np.float64),
                q_norm=g("q_norm").view(np.float32).astype(np.float64),
                k_norm=g("k_norm").view(np.float32).astype(np.float64),
                wq=wqkv[:QD], wk=wqkv[QD:QD + KVD], wv=wqkv[QD + KVD:],
                wo=np_dq(c["type_attn"], g("wo"), H, QD),
                router=g("router").view(np.float32).astype(np.float64).reshape(E, H),
                gate=[np_dq(c["type_gate_up"], g("gate")[e * sgu:(e + 1) * sgu], F, H) for e in range(E)],
                up=[np_dq(c["type_gate_up"], g("up")[e * sgu:(e + 1) * sgu], F, H) for e in range(E)],
                down=[np_dq(c["type_down"], g("down")[e * sdn:(e + 1) * sdn], H, F) for e in range(E)],
            ))
        self.kc = [[] for _ in layers]
        self.vc = [[] for _ in layers]
        self.hidden = []

    @staticmethod
    def rms(x, w, eps):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    def rope(self, v, pos):
        D = v.shape[-1]
        i = np.arange(D // 2)
        th = pos * self.c["rope_base"] ** (-2.0 * i / D)
        c, s = np.cos(th), np.sin(th)
        a, b = v[..., :D // 2], v[..., D // 2:]
        return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)

    def step(self, tok):
        c = self.c
        D, nh, nkv = c["head_dim"], c["n_head"], c["n_head_kv"]
        eps = c["rms_eps"]
        x = self.embd[tok].copy()
        pos = len(self.kc[0])
        self.hidden = []
        self.topk = []
        for il, L in enumerate(self.L):
            xn = self.rms(x, L["attn_norm"], eps)
            q = (L["wq"] @ xn).reshape(nh, D)
            k = (L["wk"] @ xn).reshape(nkv, D)
            v = (L["wv"] @ xn).reshape(nkv, D)
            q = self.rope(np.stack([self.rms(h, L["q_norm"], eps) for h in q]), pos)
            k = self.rope(np.stack([self.rms(h, L["k_norm"], eps) for h in k]), pos)
            # the cache holds f16 values
            self.kc[il].append(k.astype(np.float16).astype(np.float64))
            self.vc[il].append(v.astype(np.float16).astype(np.float64))
            K = np.stack(self.kc[il])  # [pos+1, nkv, D]
            V = np.stack(self.vc[il])
            ctx = np.empty((nh, D))
            for h in range(nh):
                kvh = h // (nh // nkv)
                s = K[:, kvh, :] @ q[h] / np.sqrt(D)
                a = np.exp(s - s.max())
                a /= a.sum()
                ctx[h] = a @ V[:, kvh, :]
            x = x + L["wo"] @ ctx.reshape(-1)
            hx = self.rms(x, L["ffn_norm"], eps)
            logits = L["router"] @ hx
            p = np.exp(logits - logits.max())
            p /= p.sum()
            order = sorted(range(len(p)), key=lambda e: (-p[e], e))[:c["n_expert_used"]]
            w = p[order] / p[order].sum()
            self.topk.append(order)
            out = np.zeros_like(x)
            for e, we in sorted(zip(order, w)):
                g = L["gate"][e] @ hx
                u = L["up"][e] @ hx
                out += we * (L["down"][e] @ (g / (1 + np.exp(-g)) * u))
            x = x + out
            self.hidden.append(x.copy())
        return self.head @ self.rms(x, self.onorm, eps)


@pytest.mark.parametrize("over", [dict(), dict(type_down=O.TYPE_Q6_K, type_head=O.TYPE_Q6_K)])
def test_oracle_model_vs_numpy_float64(over):
    cfg = dict(TINY, **over)
    oc = O.make_config(**cfg)
    om = O.OracleModel(oc, seed=5, threads=2)
    full = oc.as_dict()
    npm = NpModel(full, om.image().copy())
    for t, tok in enumerate([3, 100, 7, 511, 42, 42]):
        lw = om.forward([tok])
        ln = npm.step(tok)
        assert rel_rmse(lw, ln) < 1e-4, t
        for il in range(cfg["n_layer"]):
            assert rel_rmse(om.hidden(il), npm.hidden[il]) < 1e-4, (t, il)
            assert list(om.topk(il)[0]) == list(npm.topk[il]), (t, il)


def test_router_ties_go_to_lower_index():
    """Two identical router rows give identical probabilities: the lower expert
    index is chosen first (repeated strict-'>' argmax, model.cpp:442-451)."""
    H, F, E, K = 256, 256, 8, 3
    rng = np.random.default_rng(0)
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    hx = rng.standard_normal(H).astype(np.float32)
    best = int(np.argmax(router @ hx))
    twin = (best + 3) % E
    router[twin] = router[best]
    gate = np.concatenate([O.synth_tensor(O.tensor_key(0, 0, "gate", e), O.TYPE_Q4_K, H, F) for e in range(E)])
    up = np.concatenate([O.synth_tensor(O.tensor_key(0, 0, "up", e), O.TYPE_Q4_K, H, F) for e in range(E)])
    down = np.concatenate([O.synth_tensor(O.tensor_key(0, 0, "down", e), O.TYPE_Q4_K, F, H) for e in range(E)])
    out, logits, ti, tw = O.moe(hx, router, gate, up, down, H, F, E, K)
    assert logits[0, best] == logits[0, twin]
    lo, hi = min(best, twin), max(best, twin)
    assert list(ti[0, :2]) == [lo, hi]
    assert tw[0, 0] == tw[0, 1]
    assert abs(float(tw[0].sum()) - 1.0) < 1e-6


def f16_ulps(a, b):
    """Distance in f16 ulps between two arrays of f16 bit patterns (same sign)."""
    ia, ib = a.astype(np.int32), b.astype(np.int32)
    ia = np.where(ia & 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib & 0x8000, 0x8000 - ib, ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("over", [dict(), dict(type_down=O.TYPE_Q6_K, type_head=O.TYPE_Q6_K)])
def test_oracle_prefill_vs_numpy_float64(over):
    """One forward call over a prompt (all rows through each weight, causal
    attention over a cache appended for every row first) against the float64
    model fed the same tokens one at a time, which is what the causal mask
    means: a row attending to a later row, a row reading another row's
    position or a missing append moves the logits far outside 1e-4."""
    cfg = dict(TINY, **over)
    oc = O.make_config(**cfg)
    om = O.OracleModel(oc, seed=5, threads=2)
    npm = NpModel(oc.as_dict(), om.image().copy())
    prompt = [3, 100, 7, 511, 42, 42, 9]
    lw = om.forward(prompt)
    for tok in prompt:
        ln = npm.step(tok)
    assert om.pos == len(prompt)
    assert rel_rmse(lw, ln) < 1e-4
    for il in range(cfg["n_layer"]):
        assert rel_rmse(om.hidden(il), npm.hidden[il]) < 1e-4, il  # (~3e-5 from f16 flips)
        assert list(om.topk(il)[0]) == list(npm.topk[il]), il
    # a decode step after the prefill continues from its cache
    assert rel_rmse(om.forward([17]), npm.step(17)) < 1e-4


def test_oracle_prefill_matches_single_steps_and_split_calls():
    """Splitting a prompt over two forward calls changes nothing but the m > 1
    matmul's per-call grouping: logits and hidden states agree to ~1e-6 and
    the caches to an f16 ulp.  Single-token steps round differently (the fused
    dot of the m == 1 matmul, and the f16 cache roundings that follow from it
    flip), so they agree only to ~1e-4; both are pinned against the float64
    model above.  n == 1 is the single-token step bit for bit."""
    oc = O.make_config(**TINY)
    prompt = [5, 6, 7, 8, 300, 301, 2, 1, 0, 77]
    a = O.OracleModel(oc, seed=9, threads=2)
    b = O.OracleModel(oc, seed=9, threads=2, image=a.image())
    s = O.OracleModel(oc, seed=9, threads=2, image=a.image())
    la = a.forward(prompt)
    b.forward(prompt[:6])
    lb = b.forward(prompt[6:])
    ls = s.forward_steps(prompt)
    assert a.pos == b.pos == s.pos == len(prompt)
    assert rel_rmse(la, lb) < 1e-5
    assert rel_rmse(la, ls) < 3e-4
    n = len(prompt)
    for il in range(TINY["n_layer"]):
        assert rel_rmse(a.hidden(il), b.hidden(il)) < 1e-5
        assert rel_rmse(a.hidden(il), s.hidden(il)) < 3e-4
    for x, y in zip(a.kv(), b.kv()):
        assert f16_ulps(x[:, :, :n], y[:, :, :n]).max() <= 1
    t1 = O.OracleModel(oc, seed=9, threads=2, image=a.image())
    t2 = O.OracleModel(oc, seed=9, threads=2, image=a.image())
    assert np.array_equal(t1.forward([42]), t2.forward_steps([42]))


def test_oracle_prefill_errors():
    oc = O.make_config(**TINY)
    om = O.OracleModel(oc, seed=1, threads=1)
    with pytest.raises(RuntimeError, match="context exhausted"):
        om.forward(list(range(TINY["n_ctx"] + 1)))
    with pytest.raises(RuntimeError, match="out of range"):
        om.forward([1, TINY["n_vocab"]])
