"""GPU: knj_moe_decode_layer_noalloc (scratch in the library's fixed device
array, no allocation) against knj_moe_decode_layer (library-allocated scratch)
on the same inputs: bit-identical outputs, routing and logits on calls in a
row, each smaller than the one before, for Q4_K and Q6_K expert down; shapes
beyond the fixed array are refused; a call captured into a HIP graph replays
to the same bits.

Before every compared call, both scratches are filled with NaN by a call of
the same entry point on a NaN input of the largest compared shape (hx, act
and the logits all come out NaN), so a kernel that read scratch it had not
written in the compared call would give non-finite or different results."""
import ctypes as C

import numpy as np
import pytest

import kanjoos_amd as K
import oracle as O

pytestmark = pytest.mark.gpu

# (n_embd, n_ff, n_expert, k, seed, type_down): the largest first
SHAPES = [(2048, 768, 128, 8, 0, K.TYPE_Q4_K), (2048, 768, 64, 8, 5, K.TYPE_Q6_K),
          (1024, 512, 64, 4, 9, K.TYPE_Q4_K)]


def layer(n_embd, n_ff, n_expert, seed, type_down):
    x = O.synth_f32(O.tensor_key(seed, 0, "input"), n_embd)
    router = O.synth_tensor(O.tensor_key(seed, 0, "router"), K.TYPE_F32, n_embd, n_expert)
    gate = np.concatenate([O.synth_tensor(O.tensor_key(seed, 0, "gate", e), K.TYPE_Q4_K, n_embd, n_ff)
                           for e in range(n_expert)])
    up = np.concatenate([O.synth_tensor(O.tensor_key(seed, 0, "up", e), K.TYPE_Q4_K, n_embd, n_ff)
                         for e in range(n_expert)])
    down = np.concatenate([O.synth_tensor(O.tensor_key(seed, 0, "down", e), type_down, n_ff, n_embd)
                           for e in range(n_expert)])
    resid = O.synth_f32(O.tensor_key(seed, 0, "input", 3), n_embd)
    return x, router, gate, up, down, resid


def device_layer(n_embd, n_ff, n_expert, seed, type_down):
    x, router, gate, up, down, resid = layer(n_embd, n_ff, n_expert, seed, type_down)
    return {n: K.DeviceBuffer.from_array(a) for n, a in
            dict(x=x, router=router, gate=gate, up=up, down=down, resid=resid,
                 ones=np.ones(n_embd, np.float32)).items()}


class Outputs:
    def __init__(self, n_embd, n_expert, k):
        self.out = K.DeviceBuffer(4 * n_embd)
        self.logits = K.DeviceBuffer(4 * n_expert)
        self.ti = K.DeviceBuffer(4 * k)
        self.tw = K.DeviceBuffer(4 * k)

    def download(self):
        return (self.out.download(np.float32), self.logits.download(np.float32),
                self.ti.download(np.int32), self.tw.download(np.float32))


def call(fn, d, o, n_embd, n_ff, n_expert, k, type_down, stream=None):
    fn(d["x"], d["router"], d["gate"], d["up"], d["down"], n_embd, n_ff, n_expert, k, o.out,
       o.logits, o.ti, o.tw, norm_w=d["ones"], eps=1e-6, resid=d["resid"], type_down=type_down,
       stream=stream)


def run(fn, d, n_embd, n_ff, n_expert, k, type_down):
    o = Outputs(n_embd, n_expert, k)
    call(fn, d, o, n_embd, n_ff, n_expert, k, type_down)
    return o.download()


def poison(fn, poison_layer):
    """A call on a NaN input of the largest shape: leaves NaN in the scratch."""
    n_embd, n_ff, n_expert, k, _, type_down = SHAPES[0]
    d = dict(poison_layer)
    nan = K.DeviceBuffer.from_array(np.full(n_embd, np.nan, np.float32))
    d["x"] = nan
    o = run(fn, d, n_embd, n_ff, n_expert, k, type_down)
    assert np.all(np.isnan(o[0])) and np.all(np.isnan(o[1]))


def same_bits(a, b):
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


def test_noalloc_matches_allocating_entry_point(device):
    n_embd, n_ff, n_expert, _, seed, type_down = SHAPES[0]
    poison_layer = device_layer(n_embd, n_ff, n_expert, seed, type_down)
    for (n_embd, n_ff, n_expert, k, seed, type_down) in SHAPES:
        print(f"noalloc vs allocating: n_embd={n_embd} n_ff={n_ff} n_expert={n_expert} k={k} "
              f"down type {type_down}", flush=True)
        d = device_layer(n_embd, n_ff, n_expert, seed, type_down)
        poison(K.moe_decode_layer_noalloc, poison_layer)
        fixed = run(K.moe_decode_layer_noalloc, d, n_embd, n_ff, n_expert, k, type_down)
        poison(K.moe_decode_layer, poison_layer)
        alloc = run(K.moe_decode_layer, d, n_embd, n_ff, n_expert, k, type_down)
        for a in fixed:
            assert np.all(np.isfinite(a.astype(np.float64)))
        same_bits(fixed, alloc)
        assert len(set(fixed[2].tolist())) == k


def test_noalloc_refuses_shapes_beyond_the_fixed_array(device):
    n_embd, n_ff, n_expert, k = 2048, 4096, 16, 8  # 2048 + 8 * 4096 > 32768 floats
    bufs = {n: K.DeviceBuffer(16) for n in ("x", "router", "gate", "up", "down", "resid", "ones")}
    with pytest.raises(K.KnjError, match="fixed scratch"):
        run(K.moe_decode_layer_noalloc, bufs, n_embd, n_ff, n_expert, k, K.TYPE_Q4_K)


def hip():
    h = C.CDLL("libamdhip64.so")
    for name, args in [("hipStreamCreate", [C.POINTER(C.c_void_p)]),
                       ("hipStreamDestroy", [C.c_void_p]),
                       ("hipStreamBeginCapture", [C.c_void_p, C.c_int]),
                       ("hipStreamEndCapture", [C.c_void_p, C.POINTER(C.c_void_p)]),
                       ("hipGraphInstantiate", [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p,
                                                C.c_void_p, C.c_size_t]),
                       ("hipGraphLaunch", [C.c_void_p, C.c_void_p]),
                       ("hipStreamSynchronize", [C.c_void_p]),
                       ("hipGraphExecDestroy", [C.c_void_p]),
                       ("hipGraphDestroy", [C.c_void_p])]:
        getattr(h, name).argtypes = args
        getattr(h, name).restype = C.c_int
    return h


@pytest.mark.parametrize("shape", [0, 1])
def test_noalloc_call_replays_from_a_graph(device, shape):
    """One no-alloc call captured on a stream (relaxed capture mode); the graph
    is replayed three times, with eager calls of the allocating entry point on
    other inputs between the replays, and every replay is bit-identical to a
    direct call."""
    n_embd, n_ff, n_expert, k, seed, type_down = SHAPES[shape]
    print(f"noalloc graph: n_embd={n_embd} n_ff={n_ff} n_expert={n_expert} k={k} down type {type_down}",
          flush=True)
    d = device_layer(n_embd, n_ff, n_expert, seed, type_down)
    other = device_layer(n_embd, n_ff, n_expert, seed + 100, type_down)
    want = run(K.moe_decode_layer_noalloc, d, n_embd, n_ff, n_expert, k, type_down)
    h = hip()
    s, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert h.hipStreamCreate(C.byref(s)) == 0
    o = Outputs(n_embd, n_expert, k)
    try:
        assert h.hipStreamBeginCapture(s, 2) == 0  # hipStreamCaptureModeRelaxed
        call(K.moe_decode_layer_noalloc, d, o, n_embd, n_ff, n_expert, k, type_down, stream=s.value)
        assert h.hipStreamEndCapture(s, C.byref(graph)) == 0
        assert h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for rep in range(3):
            for b in (o.out, o.logits, o.ti, o.tw):
                b.zero()
            K.synchronize()
            assert h.hipGraphLaunch(exe, s) == 0
            assert h.hipStreamSynchronize(s) == 0
            same_bits(o.download(), want)
            # eager work between replays: the other layer through the allocating entry point
            run(K.moe_decode_layer, other, n_embd, n_ff, n_expert, k, type_down)
    finally:
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        h.hipStreamSynchronize(s)
        h.hipStreamDestroy(s)
