"""GPU: knj_moe_decode_layer_noalloc (scratch in the library's fixed device
array, no allocation) against knj_moe_decode_layer (library-allocated scratch)
on the same inputs: bit-identical outputs, routing and logits on two calls in
a row, the second smaller; shapes beyond the fixed array are refused."""
import numpy as np
import pytest

import kanjoos_amd as K
import oracle as O

pytestmark = pytest.mark.gpu


def layer(n_embd, n_ff, n_expert, seed):
    x = O.synth_f32(O.tensor_key(seed, 0, "input"), n_embd)
    router = O.synth_tensor(O.tensor_key(seed, 0, "router"), K.TYPE_F32, n_embd, n_expert)
    gate = np.concatenate([O.synth_tensor(O.tensor_key(seed, 0, "gate", e), K.TYPE_Q4_K, n_embd, n_ff)
                           for e in range(n_expert)])
    up = np.concatenate([O.synth_tensor(O.tensor_key(seed, 0, "up", e), K.TYPE_Q4_K, n_embd, n_ff)
                         for e in range(n_expert)])
    down = np.concatenate([O.synth_tensor(O.tensor_key(seed, 0, "down", e), K.TYPE_Q4_K, n_ff, n_embd)
                           for e in range(n_expert)])
    resid = O.synth_f32(O.tensor_key(seed, 0, "input", 3), n_embd)
    return x, router, gate, up, down, resid


def run(fn, d, n_embd, n_ff, n_expert, k):
    out = K.DeviceBuffer(4 * n_embd)
    logits = K.DeviceBuffer(4 * n_expert)
    ti = K.DeviceBuffer(4 * k)
    tw = K.DeviceBuffer(4 * k)
    fn(d["x"], d["router"], d["gate"], d["up"], d["down"], n_embd, n_ff, n_expert, k, out, logits,
       ti, tw, norm_w=d["ones"], eps=1e-6, resid=d["resid"])
    return (out.download(np.float32), logits.download(np.float32), ti.download(np.int32),
            tw.download(np.float32))


def test_noalloc_matches_allocating_entry_point(device):
    # config 1's layer, then a smaller one: the second call leaves the tail of
    # the fixed array holding the first call's values
    for (n_embd, n_ff, n_expert, k, seed) in [(2048, 768, 128, 8, 0), (1024, 512, 64, 4, 9)]:
        print(f"noalloc vs allocating: n_embd={n_embd} n_ff={n_ff} n_expert={n_expert} k={k}",
              flush=True)
        x, router, gate, up, down, resid = layer(n_embd, n_ff, n_expert, seed)
        d = {n: K.DeviceBuffer.from_array(a) for n, a in
             dict(x=x, router=router, gate=gate, up=up, down=down, resid=resid,
                  ones=np.ones(n_embd, np.float32)).items()}
        fixed = run(K.moe_decode_layer_noalloc, d, n_embd, n_ff, n_expert, k)
        alloc = run(K.moe_decode_layer, d, n_embd, n_ff, n_expert, k)
        for a, b in zip(fixed, alloc):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert len(set(fixed[2].tolist())) == k


def test_noalloc_refuses_shapes_beyond_the_fixed_array(device):
    n_embd, n_ff, n_expert, k = 2048, 4096, 16, 8  # 2048 + 8 * 4096 > 32768 floats
    bufs = {n: K.DeviceBuffer(16) for n in ("x", "router", "gate", "up", "down", "resid", "ones")}
    with pytest.raises(K.KnjError, match="fixed scratch"):
        run(K.moe_decode_layer_noalloc, bufs, n_embd, n_ff, n_expert, k)
