"""CPU: the oracle's format decoders and fused dots, pinned three ways.

1. Against the reference's own code (oracle/_ref/libknj_ref.so, compiled from the
   unmodified /root/reference/src/loader/dequant.cpp): bit-exact on random and
   constructed blocks.  Skipped where the reference tree is absent.
2. Against numpy's IEEE conversions (f16 <-> f32, bf16) on every pattern.
3. Against an independent numpy decode of the ggml block layouts written from
   the format description (not from this repo's header), and the fused-dot
   identity sum((d1 q - m1) x) = d1 sum(q x) - m1 sum(x) in float64.
"""
import numpy as np
import pytest

import oracle as O

RNG = np.random.default_rng(1234)


def ref_or_skip():
    r = O.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return r


# ------------------------------------------------------------------ f16 / bf16

def test_f16_decode_exhaustive_vs_numpy():
    L = O.lib()
    h = np.arange(65536, dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([L.knjo_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_decode_exhaustive_vs_reference():
    R = ref_or_skip()
    L = O.lib()
    for v in range(65536):
        a = np.float32(L.knjo_f16_to_f32(v)).view(np.uint32)
        b = np.float32(R.knjr_fp16_to_fp32(v)).view(np.uint32)
        assert a == b, hex(v)


@pytest.mark.filterwarnings("ignore:overflow encountered in cast")
def test_f32_to_f16_rne_vs_numpy():
    L = O.lib()
    vals = np.concatenate([
        RNG.standard_normal(20000).astype(np.float32),
        (RNG.standard_normal(5000) * 1e-5).astype(np.float32),   # f16 subnormal range
        (RNG.standard_normal(2000) * 7e4).astype(np.float32),    # overflow range
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 6.1035156e-05, 5.9604645e-08,
                  2.9802322e-08, 2.9802326e-08, np.inf, -np.inf], dtype=np.float32),
        # exact ties between neighbouring halves
        (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
    ])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([L.knjo_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_bf16_decode_is_a_shift():
    L = O.lib()
    for v in RNG.integers(0, 65536, 5000):
        if (v & 0x7F80) == 0x7F80 and (v & 0x7F):
            continue  # NaN payloads
        want = np.array([int(v) << 16], dtype=np.uint32).view(np.float32)[0]
        assert np.float32(L.knjo_bf16_to_f32(int(v))) == want


# ------------------------------------------------------------------ independent numpy decoders

def np_q4k(blocks: np.ndarray) -> np.ndarray:
    """ggml block_q4_K from its published layout: f16 d, f16 dmin, 12 bytes
    packing eight 6-bit scales/mins (j<4: low 6 bits of bytes j / j+4; j>=4:
    low/high nibble of byte j+4 plus the top 2 bits of bytes j-4 / j), 128
    bytes of codes where 32-byte group g carries sub-block 2g in low nibbles
    and 2g+1 in high nibbles.  Float64 arithmetic."""
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    s = b[:, 4:16].astype(np.int64)
    sc = np.zeros((b.shape[0], 8), np.int64)
    mn = np.zeros((b.shape[0], 8), np.int64)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        mn[:, j] = s[:, j + 4] & 63
    for j in range(4, 8):
        sc[:, j] = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
        mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = b[:, 16:].astype(np.int64).reshape(-1, 4, 32)
    out = np.zeros((b.shape[0], 256))
    for g in range(4):
        lo, hi = qs[:, g, :] & 15, qs[:, g, :] >> 4
        for sub, q in ((2 * g, lo), (2 * g + 1, hi)):
            out[:, 32 * sub:32 * sub + 32] = (d * sc[:, sub])[:, None] * q - (dmin * mn[:, sub])[:, None]
    return out.reshape(-1)


def np_q6k(blocks: np.ndarray) -> np.ndarray:
    """ggml block_q6_K: ql[128], qh[64], int8 scales[16], f16 d.  Weight i of
    half h (128 each), quarter t, position l: low 4 bits from ql[64h + l +
    32*(t%2)] (low nibble for t<2, high for t>=2), high 2 bits (qh[32h+l] >>
    2t) & 3, minus 32; scale index i // 16."""
    b = blocks.reshape(-1, 210)
    ql = b[:, :128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    out = np.zeros((b.shape[0], 256))
    for i in range(256):
        h, t, l = i // 128, (i // 32) % 4, i % 32
        byte = ql[:, 64 * h + l + 32 * (t % 2)]
        lo = (byte & 15) if t < 2 else (byte >> 4)
        hi = (qh[:, 32 * h + l] >> (2 * t)) & 3
        out[:, i] = d * sc[:, i // 16] * ((lo | (hi << 4)) - 32)
    return out.reshape(-1)


def random_blocks(type_id, n):
    size = 144 if type_id == O.TYPE_Q4_K else 210
    blk = RNG.integers(0, 256, n * size, dtype=np.uint8).reshape(n, size)
    # keep d (and dmin) finite: random f16 in a sane exponent range, incl. subnormals
    dd = (RNG.standard_normal(n) * 0.01).astype(np.float16)
    edge = np.array([0, 1e-7, -3e-6, 6e-5, 1.0, -2.0, 0.5, 65504.0 / 4096], dtype=np.float16)
    dd[:min(n, 8)] = edge[:min(n, 8)]
    if type_id == O.TYPE_Q4_K:
        blk[:, 0:2] = dd.view(np.uint8).reshape(n, 2)
        blk[:, 2:4] = np.abs(dd[::-1]).view(np.uint8).reshape(n, 2)
    else:
        blk[:, 208:210] = dd.view(np.uint8).reshape(n, 2)
    return np.ascontiguousarray(blk.reshape(-1))


@pytest.mark.parametrize("type_id", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_dequant_vs_independent_numpy(type_id):
    blocks = random_blocks(type_id, 300)
    got = O.dequant(type_id, blocks, 300 * 256).astype(np.float64)
    want = (np_q4k if type_id == O.TYPE_Q4_K else np_q6k)(blocks)
    # the f32 result is the correctly rounded float64 value (single rounding)
    assert np.array_equal(got.astype(np.float32), want.astype(np.float32))


def test_q4k_all_scale_min_packings():
    """Every 6-bit scale/min value in every sub-block position, decoded two ways."""
    n = 64 * 8
    blk = np.zeros((n, 144), np.uint8)
    blk[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[:, 2:4] = np.array([0.25], np.float16).view(np.uint8)
    blk[:, 16:] = RNG.integers(0, 256, (n, 128), dtype=np.uint8)
    for v in range(64):
        for j in range(8):
            row = blk[v * 8 + j]
            sc = [0] * 8
            mn = [0] * 8
            sc[j] = v
            mn[j] = 63 - v
            for jj in range(4):
                row[4 + jj] = (sc[jj] & 63) | ((sc[jj + 4] >> 4) << 6)
                row[8 + jj] = (mn[jj] & 63) | ((mn[jj + 4] >> 4) << 6)
                row[12 + jj] = (sc[jj + 4] & 15) | ((mn[jj + 4] & 15) << 4)
    blocks = np.ascontiguousarray(blk.reshape(-1))
    got = O.dequant(O.TYPE_Q4_K, blocks, n * 256)
    assert np.array_equal(got, np_q4k(blocks).astype(np.float32))


@pytest.mark.parametrize("type_id", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_dequant_vs_reference(type_id):
    R = ref_or_skip()
    blocks = random_blocks(type_id, 500)
    got = O.dequant(type_id, blocks, 500 * 256)
    want = np.zeros_like(got)
    R.knjr_dequant_row_f32(type_id, O._ptr(blocks), O._ptr(want), got.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("type_id,n", [(O.TYPE_Q4_K, 2048), (O.TYPE_Q4_K, 768), (O.TYPE_Q6_K, 768),
                                       (O.TYPE_Q6_K, 2048), (O.TYPE_F32, 2048), (O.TYPE_BF16, 2048)])
def test_fused_dot_vs_reference(type_id, n):
    R = ref_or_skip()
    for trial in range(20):
        if type_id in (O.TYPE_Q4_K, O.TYPE_Q6_K):
            w = random_blocks(type_id, n // 256)
        elif type_id == O.TYPE_F32:
            w = RNG.standard_normal(n).astype(np.float32).view(np.uint8)
        else:
            w = (RNG.standard_normal(n).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        x = RNG.standard_normal(n).astype(np.float32)
        a = O.dot(type_id, w, x)
        b = R.knjr_dequant_dot_f32(type_id, O._ptr(np.ascontiguousarray(w)), O._ptr(x), n)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


@pytest.mark.parametrize("type_id", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_fused_dot_identity_float64(type_id):
    """The factored dot equals dequantise-then-multiply up to f32 rounding."""
    w = O.synth_tensor(O.tensor_key(7, 0, "gate", 1), type_id, 2048, 16)
    dq = O.dequant(type_id, w, 2048 * 16).astype(np.float64).reshape(16, 2048)
    x = RNG.standard_normal(2048).astype(np.float32)
    got = O.matmul(type_id, w, 2048, 16, x)[0]
    want = dq @ x.astype(np.float64)
    scale = np.abs(dq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got - want) <= 1e-5 * scale)
