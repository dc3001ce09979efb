#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

  config1.json      one MoE layer, one token, seed 0: router logits, top-8 indices and
                    weights, and the MoE output of one layer (x ~ N(0,1), RMSNorm
                    weight 1, router f32 ~ N(0,0.02), 128 Q4_K experts).
  full_greedy.json  the 48-layer Qwen3-30B-A3B-shaped model (seed 0): 64 greedy
                    tokens after a 12-token prompt of random ids (numpy
                    default_rng(211); one forward call over the prompt, as the
                    reference's Model::forward runs it), with every step's 16
                    largest logits (ids and values), the top-1/top-2 margin and
                    the smallest margin.  The prompt was picked among 22 seeded
                    prompts for a sequence with several distinct tokens and a
                    margin well above the GPU/oracle difference: random-init
                    models fall into short repeating cycles.

The oracle restates the reference's CPU forward pass (oracle/); the weights come
from the seeded generator in include/knj_synth.h, which the GPU reproduces bit
for bit.  Usage: python tests/golden/make_golden.py [config1] [full]
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402

SEED = 0


def config1_inputs(n_embd=2048, n_ff=768, n_expert=128, type_down=O.TYPE_Q4_K, layer=0):
    x = O.synth_f32(O.tensor_key(SEED, layer, "input"), n_embd)
    router = O.synth_tensor(O.tensor_key(SEED, layer, "router"), O.TYPE_F32, n_embd, n_expert)
    gate = np.concatenate([O.synth_tensor(O.tensor_key(SEED, layer, "gate", e), O.TYPE_Q4_K, n_embd, n_ff)
                           for e in range(n_expert)])
    up = np.concatenate([O.synth_tensor(O.tensor_key(SEED, layer, "up", e), O.TYPE_Q4_K, n_embd, n_ff)
                         for e in range(n_expert)])
    down = np.concatenate([O.synth_tensor(O.tensor_key(SEED, layer, "down", e), type_down, n_ff, n_embd)
                           for e in range(n_expert)])
    return x, router, gate, up, down


def config1():
    x, router, gate, up, down = config1_inputs()
    hx = O.rmsnorm(x, np.ones(2048, np.float32), 1e-6)
    out, logits, ti, tw = O.moe(hx, router, gate, up, down, 2048, 768, 128, 8)
    return {"seed": SEED, "x_sha": _sha(x), "logits": logits[0].tolist(), "topk_idx": ti[0].tolist(),
            "topk_w": tw[0].tolist(), "out": out[0].tolist()}


def _sha(a):
    import hashlib

    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def full_prompt():
    rng = np.random.default_rng(211)
    return [int(t) for t in rng.integers(0, 151936, 12)]


def full_greedy(steps=64, prompt=None):
    prompt = full_prompt() if prompt is None else prompt
    cfg = O.make_config(n_ctx=128)
    t0 = time.time()
    om = O.OracleModel(cfg, seed=SEED)
    print(f"weights generated in {time.time() - t0:.0f} s", flush=True)
    logits = om.forward(list(prompt))
    toks, margins, top_ids, top_vals = [], [], [], []
    for i in range(steps):
        order = np.argsort(-logits, kind="stable")[:16]
        top_ids.append([int(j) for j in order])
        top_vals.append([float(logits[j]) for j in order])
        margins.append(float(logits[order[0]] - logits[order[1]]))
        tok = int(np.argmax(logits))
        toks.append(tok)
        if i + 1 < steps:
            logits = om.forward([tok])
        print(f"step {i}: token {tok} margin {margins[-1]:.4g}", flush=True)
    return {"seed": SEED, "prompt": list(prompt), "tokens": toks, "margins": margins,
            "min_margin": min(margins), "distinct_tokens": len(set(toks)),
            "top16_ids": top_ids, "top16_logits": top_vals, "config": cfg.as_dict()}


if __name__ == "__main__":
    which = sys.argv[1:] or ["config1", "full"]
    if "config1" in which:
        data = config1()
        with open(os.path.join(HERE, "config1.json"), "w") as f:
            json.dump(data, f)
    if "full" in which:
        data = full_greedy()
        with open(os.path.join(HERE, "full_greedy.json"), "w") as f:
            json.dump(data, f)
