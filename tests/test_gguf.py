"""GGUF loading (knj_gguf_probe, no device): geometry, types and the errors the
reference's Model::open raises (model.cpp:97-186), on files written by
tests/gguf_writer.py from a zero weight image of the right layout."""
import ctypes as C
import os

import numpy as np
import pytest

import kanjoos_amd as K
from gguf_writer import qwen3moe_meta, tensors_from_image, write_gguf

CFG = dict(n_layer=2, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=256, n_expert=16,
           n_expert_used=4, n_vocab=4096, n_ctx=160)


def zero_image(cfg):
    c = K.qwen3_30b_a3b(**cfg)
    lo = K.LayerOffsets()
    size = K.lib().knj_model_layer_offsets(C.byref(c), 0, C.byref(lo))
    return c, np.zeros(size, np.uint8)


@pytest.fixture
def gguf_path(tmp_path):
    c, img = zero_image(CFG)
    p = tmp_path / "m.gguf"
    write_gguf(p, qwen3moe_meta(CFG), tensors_from_image(c, img))
    return str(p)


def test_probe_reads_geometry_and_types(gguf_path):
    got = K.gguf_probe(gguf_path, 160)
    want = K.qwen3_30b_a3b(**CFG)
    for f in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_expert",
              "n_expert_used", "n_vocab", "n_ctx", "type_embd", "type_attn", "type_gate_up",
              "type_down", "type_head"):
        assert getattr(got, f) == getattr(want, f), f
    assert got.rope_base == pytest.approx(1e6)
    assert got.rms_eps == pytest.approx(1e-6)


def test_probe_q6k_mix(tmp_path):
    cfg = dict(CFG, type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K)
    c, img = zero_image(cfg)
    p = tmp_path / "q6.gguf"
    write_gguf(p, qwen3moe_meta(cfg), tensors_from_image(c, img))
    got = K.gguf_probe(str(p), 64)
    assert got.type_down == K.TYPE_Q6_K and got.type_head == K.TYPE_Q6_K


def _expect_error(path, n_ctx, fragment):
    with pytest.raises(K.KnjError) as e:
        K.gguf_probe(path, n_ctx)
    assert fragment in str(e.value), str(e.value)


def test_probe_errors(tmp_path, gguf_path):
    _expect_error(gguf_path, 50000, "trained context")
    c, img = zero_image(CFG)
    tens = tensors_from_image(c, img)
    # wrong architecture
    meta = [m if m[0] != "general.architecture" else (m[0], m[1], "llama") for m in qwen3moe_meta(CFG)]
    p = tmp_path / "arch.gguf"
    write_gguf(p, meta, tens)
    _expect_error(str(p), 160, "architecture is 'llama'")
    # a missing tensor
    p = tmp_path / "missing.gguf"
    write_gguf(p, qwen3moe_meta(CFG), [t for t in tens if t[0] != "blk.1.attn_v.weight"])
    _expect_error(str(p), 160, "'blk.1.attn_v.weight' is missing")
    # a wrong shape
    bad = [(n, (d if n != "blk.0.attn_q.weight" else [d[0], d[1] - 64]), t, b) for n, d, t, b in tens]
    p = tmp_path / "shape.gguf"
    write_gguf(p, qwen3moe_meta(CFG), bad)
    _expect_error(str(p), 160, "'blk.0.attn_q.weight' dim 1")
    # a missing metadata key
    p = tmp_path / "meta.gguf"
    write_gguf(p, [m for m in qwen3moe_meta(CFG) if not m[0].endswith("expert_count")], tens)
    _expect_error(str(p), 160, "expert_count' is missing")
    # truncated
    raw = open(gguf_path, "rb").read()
    p = tmp_path / "trunc.gguf"
    p.write_bytes(raw[: len(raw) // 2])
    _expect_error(str(p), 160, "past the end")
    # not a GGUF file
    p = tmp_path / "junk.gguf"
    p.write_bytes(b"NOPE" + os.urandom(64))
    _expect_error(str(p), 160, "bad magic")


def test_probe_corrupt_files_fail_cleanly(tmp_path):
    """Truncations and random byte changes in the header, metadata and tensor
    table of a small model's GGUF: the probe either accepts the file (a
    change that leaves it consistent) or refuses it with an error, and never
    reads out of bounds (a crash would end the test run; the same set ran
    clean under AddressSanitizer)."""
    cfg = dict(n_layer=1, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=256, n_expert=8,
               n_expert_used=2, n_vocab=512, n_ctx=64)
    c, img = zero_image(cfg)
    base = tmp_path / "base.gguf"
    write_gguf(base, qwen3moe_meta(cfg), tensors_from_image(c, img))
    raw = base.read_bytes()
    head = min(len(raw), 6000)
    rng = np.random.default_rng(7)
    p = tmp_path / "bad.gguf"
    accepted = refused = 0
    cases = [raw[:int(n)] for n in rng.integers(0, head, 60)]
    for _ in range(200):
        b = bytearray(raw)
        for pos in rng.integers(0, head, int(rng.integers(1, 6))):
            b[int(pos)] = int(rng.integers(0, 256))
        cases.append(bytes(b))
    for data in cases:
        p.write_bytes(data)
        try:
            K.gguf_probe(str(p), 64)
            accepted += 1
        except K.KnjError:
            refused += 1
    assert refused >= 60 and accepted + refused == len(cases)


@pytest.mark.gpu
@pytest.mark.parametrize("cfgkw", [dict(), dict(type_down=K.TYPE_Q6_K, type_head=K.TYPE_Q6_K)])
def test_gguf_roundtrip_model(device, tmp_path, cfgkw):
    """A synthetic model's weights written out as a GGUF file and loaded back:
    the device image is byte-identical and decode gives identical logits and
    greedy tokens."""
    cfg = dict(CFG, **cfgkw)
    print(f"gguf round trip {cfg}", flush=True)
    a = K.Model.synthetic(K.qwen3_30b_a3b(**cfg), seed=3)
    img = a.download_image()
    p = tmp_path / "rt.gguf"
    write_gguf(p, qwen3moe_meta(cfg), tensors_from_image(a.cfg, img))
    b = K.Model.from_gguf(str(p), cfg["n_ctx"])
    try:
        got = b.download_image()
        assert got.size == img.size
        bad = np.flatnonzero(got != img)
        assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"
        la, lb = a.forward([5, 6, 7]), b.forward([5, 6, 7])
        assert np.array_equal(la, lb)
        first = int(np.argmax(la))
        assert list(a.decode_greedy(first, 16)) == list(b.decode_greedy(first, 16))
    finally:
        a.close()
        b.close()


@pytest.mark.gpu
def test_cpp_driver_gguf(device, tmp_path):
    """kanjoos-run --model (knj::Model::open) on a GGUF file written from the
    synthetic weights prints the same tokens as kanjoos-run on those weights."""
    import subprocess

    a = K.Model.synthetic(K.qwen3_30b_a3b(**CFG), seed=5)
    p = tmp_path / "drv.gguf"
    write_gguf(p, qwen3moe_meta(CFG), tensors_from_image(a.cfg, a.download_image()))
    a.close()
    exe = os.path.join(os.path.dirname(K.LIB_PATH), "kanjoos-run")
    common = ["--ctx", "64", "--prompt", "8", "--n-predict", "16", "--seed", "5"]
    outs = []
    for extra in (["--model", str(p)], ["--small", "--layers", "2"]):
        r = subprocess.run([exe] + extra + common, capture_output=True, text=True, timeout=60)
        print(r.stdout + r.stderr, flush=True)
        assert r.returncode == 0
        outs.append(r.stdout.strip().splitlines()[-1])
    assert outs[0].startswith("tokens:") and outs[0] == outs[1]


def test_cpp_driver_gguf_error(tmp_path):
    """A broken file is refused with the loader's message and a nonzero exit,
    before any device work (the reference's main.cpp reports open errors)."""
    import subprocess

    exe = os.path.join(os.path.dirname(K.LIB_PATH), "kanjoos-run")
    if not os.path.exists(exe):
        pytest.skip("kanjoos-run not built")
    p = tmp_path / "junk.gguf"
    p.write_bytes(b"GGUF" + bytes(40))
    r = subprocess.run([exe, "--model", str(p)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 3 and "model:" in r.stderr, (r.returncode, r.stderr)
