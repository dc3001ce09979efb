"""CPU oracle for the Kanjoos MoE decode path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the thing timed on the host).  The GPU product path never routes
through it.

``oracle/libknj_oracle.so`` restates the reference's CPU forward pass
(/root/reference/src/model/model.cpp, src/loader/dequant.cpp) in the reference's
own order of floating-point operations; ``oracle/_ref/libknj_ref.so`` (built
from the reference's unmodified dequant sources when /root/reference exists) is
used to pin the restatement's format decoders and fused dots.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libknj_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libknj_ref.so")

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K, TYPE_BF16 = 0, 1, 12, 14, 30
KIND = dict(embd=1, head=2, q=3, k=4, v=5, o=6, router=7, gate=8, up=9, down=10, input=11)


class ModelConfig(C.Structure):
    """Mirror of ``knj_model_config`` (include/knj_model.h)."""

    _fields_ = [
        ("n_layer", C.c_int32), ("n_embd", C.c_int32), ("n_head", C.c_int32),
        ("n_head_kv", C.c_int32), ("head_dim", C.c_int32), ("n_ff", C.c_int32),
        ("n_expert", C.c_int32), ("n_expert_used", C.c_int32), ("n_vocab", C.c_int32),
        ("n_ctx", C.c_int32), ("rms_eps", C.c_float), ("rope_base", C.c_float),
        ("type_embd", C.c_int32), ("type_attn", C.c_int32), ("type_gate_up", C.c_int32),
        ("type_down", C.c_int32), ("type_head", C.c_int32), ("init_std", C.c_float),
    ]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


def make_config(**kw) -> ModelConfig:
    """Qwen3-30B-A3B geometry by default; override any field."""
    base = dict(n_layer=48, n_embd=2048, n_head=32, n_head_kv=4, head_dim=128, n_ff=768,
                n_expert=128, n_expert_used=8, n_vocab=151936, n_ctx=4352, rms_eps=1e-6,
                rope_base=1e6, type_embd=TYPE_BF16, type_attn=TYPE_Q4_K,
                type_gate_up=TYPE_Q4_K, type_down=TYPE_Q4_K, type_head=TYPE_BF16,
                init_std=0.02)
    base.update(kw)
    return ModelConfig(**base)


def row_bytes(type_id: int, n: int) -> int:
    if type_id == TYPE_F32:
        return 4 * n
    if type_id in (TYPE_F16, TYPE_BF16):
        return 2 * n
    if type_id == TYPE_Q4_K:
        return n // 256 * 144
    if type_id == TYPE_Q6_K:
        return n // 256 * 210
    raise ValueError(type_id)


def build(ref: bool = True) -> None:
    """Compile the oracle (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all" if ref else "oracle"], check=True)


_lib = None
_ref = None
_P = C.c_void_p
_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = C.CDLL(LIB_PATH)
        L.knjo_f16_to_f32.restype = C.c_float
        L.knjo_f16_to_f32.argtypes = [C.c_uint16]
        L.knjo_f32_to_f16.restype = C.c_uint16
        L.knjo_f32_to_f16.argtypes = [C.c_float]
        L.knjo_bf16_to_f32.restype = C.c_float
        L.knjo_bf16_to_f32.argtypes = [C.c_uint16]
        L.knjo_dequant_row_f32.argtypes = [C.c_int, _P, _P, C.c_uint64]
        L.knjo_dequant_dot_f32.restype = C.c_float
        L.knjo_dequant_dot_f32.argtypes = [C.c_int, _P, _P, C.c_uint64]
        L.knjo_tensor_key.restype = C.c_uint64
        L.knjo_tensor_key.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int]
        L.knjo_synth_tensor.argtypes = [C.c_uint64, C.c_int, C.c_uint64, C.c_uint64, C.c_float, _P, C.c_int]
        L.knjo_synth_model.argtypes = [C.POINTER(ModelConfig), C.c_uint64, _P, C.c_int]
        L.knjo_matmul.argtypes = [C.c_int, _P, C.c_int, C.c_int, _P, C.c_int, _P, C.c_int]
        L.knjo_moe.argtypes = [_P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P,
                               C.c_int, C.c_int, _P, _P, _P, _P, C.c_int]
        L.knjo_rmsnorm.argtypes = [_P, _P, _P, C.c_int, C.c_float]
        L.knjo_model_create.restype = _P
        L.knjo_model_create.argtypes = [C.POINTER(ModelConfig), C.c_uint64, _P, C.c_int]
        L.knjo_model_free.argtypes = [_P]
        L.knjo_model_image.restype = _P
        L.knjo_model_image.argtypes = [_P]
        L.knjo_model_image_bytes.restype = C.c_uint64
        L.knjo_model_image_bytes.argtypes = [_P]
        L.knjo_model_reset.argtypes = [_P]
        L.knjo_model_pos.restype = C.c_int
        L.knjo_model_pos.argtypes = [_P]
        L.knjo_model_threads.restype = C.c_int
        L.knjo_model_threads.argtypes = [_P]
        L.knjo_model_forward.restype = C.c_int
        L.knjo_model_forward.argtypes = [_P, _P, C.c_int, _P]
        L.knjo_model_forward_steps.restype = C.c_int
        L.knjo_model_forward_steps.argtypes = [_P, _P, C.c_int, _P]
        L.knjo_model_hidden.restype = _f32p
        L.knjo_model_hidden.argtypes = [_P, C.c_int]
        L.knjo_model_topk_idx.restype = C.POINTER(C.c_int32)
        L.knjo_model_topk_idx.argtypes = [_P, C.c_int]
        L.knjo_model_topk_w.restype = _f32p
        L.knjo_model_topk_w.argtypes = [_P, C.c_int]
        L.knjo_model_kv_k.restype = C.POINTER(C.c_uint16)
        L.knjo_model_kv_k.argtypes = [_P]
        L.knjo_model_kv_v.restype = C.POINTER(C.c_uint16)
        L.knjo_model_kv_v.argtypes = [_P]
        L.knjo_model_set_pos.restype = C.c_int
        L.knjo_model_set_pos.argtypes = [_P, C.c_int]
        L.knjo_model_set_kv_source.argtypes = [_P, _P, _P]
        L.knjo_model_kv_rms.argtypes = [_P, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.knjo_model_kv_rms.restype = None
        L.knjo_model_kv_stats.argtypes = [_P, C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                          C.POINTER(C.c_int), C.POINTER(C.c_float)]
        L.knjo_last_error.restype = C.c_char_p
        _lib = L
    return _lib


def ref():
    """The reference's own dequant code (oracle/_ref), or None when it is not built."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_PATH):
            return None
        R = C.CDLL(REF_PATH)
        R.knjr_fp16_to_fp32.restype = C.c_float
        R.knjr_fp16_to_fp32.argtypes = [C.c_uint16]
        R.knjr_bf16_to_fp32.restype = C.c_float
        R.knjr_bf16_to_fp32.argtypes = [C.c_uint16]
        R.knjr_dequant_row_f32.argtypes = [C.c_int, _P, _P, C.c_uint64]
        R.knjr_dequant_dot_f32.restype = C.c_float
        R.knjr_dequant_dot_f32.argtypes = [C.c_int, _P, _P, C.c_uint64]
        _ref = R
    return _ref


# ------------------------------------------------------------------ helpers

def tensor_key(seed: int, layer: int, kind: str, expert: int = -1) -> int:
    return lib().knjo_tensor_key(seed, layer, KIND[kind], expert)


def synth_tensor(key: int, type_id: int, n_in: int, n_rows: int, std: float = 0.02,
                 threads: int = 0) -> np.ndarray:
    out = np.zeros(row_bytes(type_id, n_in) * n_rows, dtype=np.uint8)
    lib().knjo_synth_tensor(key, type_id, n_in, n_rows, std, _ptr(out), threads)
    return out


def synth_f32(key: int, n: int, std: float = 1.0) -> np.ndarray:
    return synth_tensor(key, TYPE_F32, n, 1, std).view(np.float32).copy()


def dequant(type_id: int, blob: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().knjo_dequant_row_f32(type_id, _ptr(np.ascontiguousarray(blob)), _ptr(out), n)
    return out


def dot(type_id: int, blob: np.ndarray, x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().knjo_dequant_dot_f32(type_id, _ptr(np.ascontiguousarray(blob)), _ptr(x), x.size)


def matmul(type_id: int, w: np.ndarray, n_in: int, n_out: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n_in)
    y = np.zeros((x.shape[0], n_out), dtype=np.float32)
    lib().knjo_matmul(type_id, _ptr(w), n_in, n_out, _ptr(x), x.shape[0], _ptr(y), threads)
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    lib().knjo_rmsnorm(_ptr(x), _ptr(np.ascontiguousarray(w, dtype=np.float32)), _ptr(out), x.size, eps)
    return out


def moe(hx, router_w, gate, up, down, n_embd, n_ff, n_expert, k, type_gu=TYPE_Q4_K,
        type_down=TYPE_Q4_K, threads: int = 0):
    """Model::moe on m rows; returns (out, logits, topk_idx, topk_w)."""
    hx = np.ascontiguousarray(hx, dtype=np.float32).reshape(-1, n_embd)
    m = hx.shape[0]
    out = np.zeros((m, n_embd), np.float32)
    logits = np.zeros((m, n_expert), np.float32)
    ti = np.zeros((m, k), np.int32)
    tw = np.zeros((m, k), np.float32)
    lib().knjo_moe(_ptr(hx), m, n_embd, n_ff, n_expert, k, _ptr(router_w), _ptr(gate), _ptr(up),
                   _ptr(down), type_gu, type_down, _ptr(out), _ptr(logits), _ptr(ti), _ptr(tw),
                   threads)
    return out, logits, ti, tw


class OracleModel:
    """Model-shaped wrapper (open/forward/reset/pos) over the oracle library."""

    def __init__(self, cfg: ModelConfig, seed: int = 0, image: np.ndarray | None = None,
                 threads: int = 0):
        self.cfg = cfg
        self._image = image  # keep the caller's buffer alive
        L = lib()
        self.h = L.knjo_model_create(C.byref(cfg), seed, _ptr(image) if image is not None else None,
                                     threads)
        if not self.h:
            raise RuntimeError(L.knjo_last_error().decode())

    def close(self):
        if self.h:
            lib().knjo_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self) -> int:
        return lib().knjo_model_pos(self.h)

    @property
    def threads(self) -> int:
        return lib().knjo_model_threads(self.h)

    def image(self) -> np.ndarray:
        """The weight image as a view (no copy): valid while this model is alive."""
        L = lib()
        n = L.knjo_model_image_bytes(self.h)
        p = L.knjo_model_image(self.h)
        return np.ctypeslib.as_array(C.cast(p, _u8p), shape=(n,))

    def reset(self):
        lib().knjo_model_reset(self.h)

    def forward(self, tokens) -> np.ndarray:
        """One Model::forward call over all of `tokens` (the batched prefill)."""
        return self._run(lib().knjo_model_forward, tokens)

    def forward_steps(self, tokens) -> np.ndarray:
        """`tokens` as single-token forward calls, one after another."""
        return self._run(lib().knjo_model_forward_steps, tokens)

    def _run(self, fn, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        logits = np.zeros(self.cfg.n_vocab, dtype=np.float32)
        if fn(self.h, _ptr(t), t.size, _ptr(logits)) != 0:
            raise RuntimeError(lib().knjo_last_error().decode())
        return logits

    def hidden(self, il: int) -> np.ndarray:
        p = lib().knjo_model_hidden(self.h, il)
        return np.ctypeslib.as_array(p, shape=(self.cfg.n_embd,)).copy()

    def topk(self, il: int):
        k = self.cfg.n_expert_used
        i = np.ctypeslib.as_array(lib().knjo_model_topk_idx(self.h, il), shape=(k,)).copy()
        w = np.ctypeslib.as_array(lib().knjo_model_topk_w(self.h, il), shape=(k,)).copy()
        return i, w

    def kv(self):
        """(K, V) f16 caches as uint16 views [n_layer][n_head_kv][n_ctx][head_dim]."""
        c = self.cfg
        shape = (c.n_layer, c.n_head_kv, c.n_ctx, c.head_dim)
        k = np.ctypeslib.as_array(lib().knjo_model_kv_k(self.h), shape=shape)
        v = np.ctypeslib.as_array(lib().knjo_model_kv_v(self.h), shape=shape)
        return k, v

    def set_kv_source(self, k: np.ndarray | None, v: np.ndarray | None):
        """Adopt these f16 caches' values for newly written slots (see the C header)."""
        self._kv_src = (k, v)
        lib().knjo_model_set_kv_source(self.h, _ptr(k) if k is not None else None,
                                       _ptr(v) if v is not None else None)

    def kv_stats(self):
        a, d, u, mid = C.c_int64(), C.c_int64(), C.c_int(), C.c_float()
        lib().knjo_model_kv_stats(self.h, C.byref(a), C.byref(d), C.byref(u), C.byref(mid))
        d2, v2 = C.c_double(), C.c_double()
        lib().knjo_model_kv_rms(self.h, C.byref(d2), C.byref(v2))
        rel = (d2.value / v2.value) ** 0.5 if v2.value > 0 else 0.0
        return dict(adopted=a.value, differing=d.value, max_ulp=u.value, max_mid_dist=mid.value,
                    rel_rms_dist=rel)

    def set_pos(self, pos: int):
        if lib().knjo_model_set_pos(self.h, pos) != 0:
            raise ValueError(pos)

    def greedy(self, prompt, steps: int):
        """Greedy decode: argmax with the first maximum winning (main.cpp:126-132)."""
        logits = self.forward(prompt)
        out = []
        for i in range(steps):
            tok = int(np.argmax(logits))  # numpy returns the first maximum
            out.append(tok)
            if i + 1 < steps:
                logits = self.forward([tok])
        return out
