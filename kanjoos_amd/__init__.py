"""kanjoos_amd -- MI355X (gfx950) batch-1 MoE decode path of Kanjoos.

Python view of the C ABI in ``include/knj_capi.h`` (``libkanjoos_amd.so``,
built in-tree by ``kanjoos_amd/build.py``).  The classes mirror the reference's
host interfaces:

* :class:`Model` -- ``knj::Model`` (/root/reference/src/model/model.h:55-80):
  ``forward(tokens) -> logits`` of the last token, ``reset()``, ``pos``.
* :func:`open_device` -- the C2 gate (``Backend::create``,
  /root/reference/src/device/backend.cpp:54-62): refuses a non-gfx950 device.

There is no CPU fallback: every call goes to the HIP library, and importing a
missing library raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkanjoos_amd.so")

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K, TYPE_BF16 = 0, 1, 12, 14, 30
KNJ_OK, KNJ_E_CORRECTNESS, KNJ_E_ARCH, KNJ_E_ENV, KNJ_E_HIP, KNJ_E_ARG, KNJ_E_STATE = 0, 5, 6, 7, 9, 22, 23

# every entry point include/knj_capi.h declares
EXPORTS = (
    "knj_device_open", "knj_device_close", "knj_device_caps_get", "knj_check_arch",
    "knj_built_arch", "knj_last_error", "knj_malloc", "knj_free", "knj_memcpy_h2d",
    "knj_memcpy_d2h", "knj_memset_zero", "knj_synchronize", "knj_dequant", "knj_gemv",
    "knj_rmsnorm", "knj_moe_router", "knj_moe_decode_layer", "knj_moe_decode_layer_noalloc", "knj_moe_batch_layer", "knj_attention_step", "knj_model_create_synthetic", "knj_model_create_from_image",
    "knj_model_free", "knj_model_image_bytes", "knj_model_image_device", "knj_model_layer_offsets", "knj_model_fill_kv", "knj_gguf_probe",
    "knj_model_create_from_gguf", "knj_model_config_get",
    "knj_model_download_image", "knj_model_reset", "knj_model_pos", "knj_model_set_pos",
    "knj_model_forward", "knj_model_decode_greedy", "knj_model_hidden", "knj_model_topk",
    "knj_model_logits", "knj_model_kv_download", "knj_model_kv_upload",
    "knj_model_time_decode", "knj_model_time_experts", "knj_model_profile",
    "knj_model_transfer_bytes", "knj_device_floor",
    "knj_batch_create", "knj_batch_free", "knj_batch_pos", "knj_batch_forward",
    "knj_batch_decode_greedy", "knj_batch_fill_kv", "knj_batch_hidden", "knj_batch_topk",
    "knj_batch_kv_download", "knj_batch_kv_upload", "knj_batch_set_pos",
)


class KnjError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[knj {code}] {msg}")
        self.code = code


class ModelConfig(C.Structure):
    """``knj_model_config`` (include/knj_model.h)."""

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


def qwen3_30b_a3b(**kw) -> ModelConfig:
    """Qwen3-30B-A3B geometry: 48 layers, hidden 2048, 32/4 heads x 128, 128 experts
    top-8 of width 768, vocab 151936, Q4_K attention and experts, bf16 embeddings
    and LM head.  Any field can be overridden."""
    base = dict(n_layer=48, n_embd=2048, n_head=32, n_head_kv=4, head_dim=128, n_ff=768,
                n_expert=128, n_expert_used=8, n_vocab=151936, n_ctx=4352, rms_eps=1e-6,
                rope_base=1e6, type_embd=TYPE_BF16, type_attn=TYPE_Q4_K,
                type_gate_up=TYPE_Q4_K, type_down=TYPE_Q4_K, type_head=TYPE_BF16,
                init_std=0.02)
    base.update(kw)
    return ModelConfig(**base)


class LayerOffsets(C.Structure):
    """Byte offsets of one layer's tensors in the weight image (knj_layer_offsets)."""
    _fields_ = [(n, C.c_uint64) for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm", "wqkv", "wo",
                                           "router", "gate", "up", "down")]


class Span(C.Structure):
    """One profiled kernel launch (include/knj_capi.h knj_span)."""
    _fields_ = [("name", C.c_char * 32), ("kernel", C.c_char * 40), ("layer", C.c_int32),
                ("stream", C.c_int32), ("start_ns", C.c_uint64), ("end_ns", C.c_uint64)]


class DeviceCaps(C.Structure):
    _fields_ = [
        ("gcn_arch", C.c_char * 32), ("name", C.c_char * 64), ("wave_size", C.c_int32),
        ("cu_count", C.c_int32), ("clock_khz", C.c_int32), ("lds_per_block", C.c_int32),
        ("l2_bytes", C.c_int32), ("arch_ok", C.c_int32), ("has_mfma_bf16", C.c_int32),
        ("has_mfma_i8", C.c_int32), ("has_fp8", C.c_int32), ("vram_total", C.c_uint64),
        ("vram_free", C.c_uint64),
    ]


_P = C.c_void_p
_i = C.c_int
_f = C.c_float
_u64 = C.c_uint64
_SIGS = {
    "knj_device_open": (_i, [_i]),
    "knj_device_close": (_i, []),
    "knj_device_caps_get": (_i, [C.POINTER(DeviceCaps)]),
    "knj_check_arch": (_i, [C.c_char_p, C.c_char_p, C.c_char_p]),
    "knj_built_arch": (C.c_char_p, []),
    "knj_last_error": (C.c_char_p, []),
    "knj_malloc": (_i, [C.POINTER(_P), _u64]),
    "knj_free": (_i, [_P]),
    "knj_memcpy_h2d": (_i, [_P, _P, _u64]),
    "knj_memcpy_d2h": (_i, [_P, _P, _u64]),
    "knj_memset_zero": (_i, [_P, _u64]),
    "knj_synchronize": (_i, []),
    "knj_dequant": (_i, [_i, _P, _u64, _P, _P]),
    "knj_gemv": (_i, [_i, _P, _i, _i, _P, _P, _f, _P, _P, _P]),
    "knj_rmsnorm": (_i, [_P, _P, _i, _f, _P, _P]),
    "knj_moe_router": (_i, [_P, _P, _f, _P, _i, _i, _i, _P, _P, _P, _P, _P]),
    "knj_moe_decode_layer": (_i, [_P, _P, _f, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _P, _P,
                                  _P, _P, _P, _P]),
    "knj_moe_decode_layer_noalloc": (_i, [_P, _P, _f, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _P,
                                          _P, _P, _P, _P, _P]),
    "knj_moe_batch_layer": (_i, [_P, _P, _f, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _i, _P, _P,
                                  _P, _P, _P, _P]),
    "knj_attention_step": (_i, [_P, _P, _P, _P, _P, _f, _f, _i, _i, _i, _i, _i, _P, _P, _P, _P]),
    "knj_model_create_synthetic": (_i, [C.POINTER(ModelConfig), _u64, C.POINTER(_P)]),
    "knj_model_create_from_image": (_i, [C.POINTER(ModelConfig), _P, _u64, C.POINTER(_P)]),
    "knj_model_free": (_i, [_P]),
    "knj_model_image_bytes": (_u64, [_P]),
    "knj_model_image_device": (_P, [_P]),
    "knj_model_layer_offsets": (_u64, [C.POINTER(ModelConfig), _i, C.POINTER(LayerOffsets)]),
    "knj_model_fill_kv": (_i, [_P, _i, _u64]),
    "knj_gguf_probe": (_i, [C.c_char_p, _i, C.POINTER(ModelConfig)]),
    "knj_model_create_from_gguf": (_i, [C.c_char_p, _i, C.POINTER(_P)]),
    "knj_model_config_get": (_i, [_P, C.POINTER(ModelConfig)]),
    "knj_model_download_image": (_i, [_P, _P, _u64]),
    "knj_model_reset": (_i, [_P]),
    "knj_model_pos": (_i, [_P]),
    "knj_model_set_pos": (_i, [_P, _i]),
    "knj_model_forward": (_i, [_P, _P, _i, _P]),
    "knj_model_decode_greedy": (_i, [_P, C.c_int32, _i, _P]),
    "knj_model_hidden": (_i, [_P, _i, _P]),
    "knj_model_topk": (_i, [_P, _i, _P, _P]),
    "knj_model_logits": (_i, [_P, _P]),
    "knj_model_kv_download": (_i, [_P, _P, _P]),
    "knj_model_kv_upload": (_i, [_P, _P, _P]),
    "knj_model_time_decode": (_i, [_P, _i, C.POINTER(_f)]),
    "knj_model_time_experts": (_i, [_P, _i, C.POINTER(_f), C.POINTER(_f)]),
    "knj_model_profile": (_i, [_P, C.c_int32, _i, _P, _P, _i, C.POINTER(_i), C.POINTER(_u64)]),
    "knj_model_transfer_bytes": (_i, [_P, C.POINTER(_u64), C.POINTER(_u64)]),
    "knj_device_floor": (_i, [_i, C.POINTER(_u64)]),
    "knj_batch_create": (_i, [_P, _i, _i, C.POINTER(_P)]),
    "knj_batch_free": (_i, [_P]),
    "knj_batch_pos": (_i, [_P]),
    "knj_batch_forward": (_i, [_P, _P, _P]),
    "knj_batch_decode_greedy": (_i, [_P, _P, _i, _P]),
    "knj_batch_fill_kv": (_i, [_P, _i, _u64]),
    "knj_batch_hidden": (_i, [_P, _i, _i, _P]),
    "knj_batch_topk": (_i, [_P, _i, _i, _P, _P]),
    "knj_batch_kv_download": (_i, [_P, _i, _P, _P]),
    "knj_batch_kv_upload": (_i, [_P, _i, _P, _P]),
    "knj_batch_set_pos": (_i, [_P, _i]),
}

_lib = None


def lib():
    """The HIP library.  Raises if it has not been built -- there is no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python -m kanjoos_amd.build` first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != KNJ_OK:
        raise KnjError(rc, lib().knj_last_error().decode(errors="replace"))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


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


# ------------------------------------------------------------------ device

def open_device(device: int = 0) -> DeviceCaps:
    """Arch-guarded open of `device`; returns its probed capabilities."""
    check(lib().knj_device_open(device))
    caps = DeviceCaps()
    check(lib().knj_device_caps_get(C.byref(caps)))
    return caps


def close_device() -> None:
    check(lib().knj_device_close())


def synchronize() -> None:
    check(lib().knj_synchronize())


class DeviceBuffer:
    """A device allocation of `nbytes` (HIP memory owned by this object)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _P()
        check(lib().knj_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().knj_memcpy_h2d(self.ptr, _ptr(a), a.nbytes))

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        check(lib().knj_memcpy_d2h(_ptr(out), self.ptr, out.nbytes))
        return out

    def zero(self) -> None:
        check(lib().knj_memset_zero(self.ptr, self.nbytes))

    def free(self) -> None:
        if self.ptr:
            lib().knj_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(b):
    return None if b is None else (b.ptr if isinstance(b, DeviceBuffer) else b)


# ------------------------------------------------------------------ primitives

def dequant(type_id: int, w: DeviceBuffer, n: int, out: DeviceBuffer) -> None:
    check(lib().knj_dequant(type_id, _p(w), n, _p(out), None))


def gemv(type_id: int, w, n_in: int, n_out: int, x, y, norm_w=None, eps: float = 1e-6,
         resid=None) -> None:
    check(lib().knj_gemv(type_id, _p(w), n_in, n_out, _p(x), _p(norm_w), eps, _p(resid), _p(y), None))


def moe_router(x, router_w, n_embd, n_expert, k, hx, logits, topk_idx, topk_w, norm_w=None,
               eps: float = 1e-6) -> None:
    check(lib().knj_moe_router(_p(x), _p(norm_w), eps, _p(router_w), n_embd, n_expert, k, _p(hx),
                               _p(logits), _p(topk_idx), _p(topk_w), None))


def moe_decode_layer(x, router_w, gate, up, down, n_embd, n_ff, n_expert, k, out, logits,
                     topk_idx, topk_w, norm_w=None, eps: float = 1e-6, resid=None,
                     type_gate_up: int = TYPE_Q4_K, type_down: int = TYPE_Q4_K,
                     stream=None) -> None:
    check(lib().knj_moe_decode_layer(_p(x), _p(norm_w), eps, _p(router_w), _p(gate), _p(up),
                                     _p(down), type_gate_up, type_down, n_embd, n_ff, n_expert, k,
                                     _p(resid), _p(out), _p(logits), _p(topk_idx), _p(topk_w),
                                     stream))


def moe_decode_layer_noalloc(x, router_w, gate, up, down, n_embd, n_ff, n_expert, k, out, logits,
                             topk_idx, topk_w, norm_w=None, eps: float = 1e-6, resid=None,
                             type_gate_up: int = TYPE_Q4_K, type_down: int = TYPE_Q4_K,
                             stream=None) -> None:
    """knj_moe_decode_layer with its scratch in the library's fixed device array
    (no allocation; n_embd + k * n_ff <= 32768)."""
    check(lib().knj_moe_decode_layer_noalloc(_p(x), _p(norm_w), eps, _p(router_w), _p(gate), _p(up),
                                             _p(down), type_gate_up, type_down, n_embd, n_ff,
                                             n_expert, k, _p(resid), _p(out), _p(logits),
                                             _p(topk_idx), _p(topk_w), stream))


def moe_batch_layer(x, router_w, gate, up, down, n_tokens, n_embd, n_ff, n_expert, k, out, logits,
                    topk_idx, topk_w, norm_w=None, eps: float = 1e-6, resid=None,
                    type_gate_up: int = TYPE_Q4_K, type_down: int = TYPE_Q4_K, stream=None) -> None:
    check(lib().knj_moe_batch_layer(_p(x), _p(norm_w), eps, _p(router_w), _p(gate), _p(up),
                                    _p(down), type_gate_up, type_down, n_tokens, n_embd, n_ff,
                                    n_expert, k, _p(resid), _p(out), _p(logits), _p(topk_idx),
                                    _p(topk_w), stream))


def device_floor(n: int = 256) -> int:
    """Mean span of `n` empty kernels timed through the profiling event path, ns."""
    v = C.c_uint64(0)
    check(lib().knj_device_floor(n, C.byref(v)))
    return v.value


def gguf_probe(path: str, n_ctx: int) -> ModelConfig:
    """Geometry and weight types of a qwen3moe GGUF file (no device needed)."""
    cfg = ModelConfig()
    check(lib().knj_gguf_probe(os.fsencode(path), n_ctx, C.byref(cfg)))
    return cfg


def attention_step(q, k, v, q_norm, k_norm, eps, rope_base, pos, n_head, n_head_kv, head_dim,
                   n_ctx, k_cache, v_cache, out) -> None:
    check(lib().knj_attention_step(_p(q), _p(k), _p(v), _p(q_norm), _p(k_norm), eps, rope_base, pos,
                                   n_head, n_head_kv, head_dim, n_ctx, _p(k_cache), _p(v_cache),
                                   _p(out), None))


# ------------------------------------------------------------------ model

class Model:
    """The device decode step, shaped like the reference's ``knj::Model``."""

    def __init__(self, handle, cfg: ModelConfig):
        self.h = handle
        self.cfg = cfg

    @classmethod
    def synthetic(cls, cfg: ModelConfig, seed: int = 0) -> "Model":
        h = _P()
        check(lib().knj_model_create_synthetic(C.byref(cfg), seed, C.byref(h)))
        return cls(h.value, cfg)

    @classmethod
    def from_gguf(cls, path: str, n_ctx: int) -> "Model":
        """A qwen3moe GGUF file (knj_model_create_from_gguf)."""
        h = _P()
        check(lib().knj_model_create_from_gguf(os.fsencode(path), n_ctx, C.byref(h)))
        cfg = ModelConfig()
        check(lib().knj_model_config_get(h.value, C.byref(cfg)))
        return cls(h.value, cfg)

    @classmethod
    def from_image(cls, cfg: ModelConfig, image: np.ndarray) -> "Model":
        image = np.ascontiguousarray(image, dtype=np.uint8)
        h = _P()
        check(lib().knj_model_create_from_image(C.byref(cfg), _ptr(image), image.nbytes, C.byref(h)))
        return cls(h.value, cfg)

    def close(self) -> None:
        if self.h:
            lib().knj_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self) -> int:
        return lib().knj_model_pos(self.h)

    def set_pos(self, pos: int) -> None:
        check(lib().knj_model_set_pos(self.h, pos))

    def reset(self) -> None:
        check(lib().knj_model_reset(self.h))

    def fill_kv(self, n_pos: int, seed: int = 0) -> None:
        """Seeded f16 values in cache slots [0, n_pos) of every layer; position = n_pos."""
        check(lib().knj_model_fill_kv(self.h, n_pos, seed))

    def image_device(self) -> int:
        """Device address of the weight image."""
        return lib().knj_model_image_device(self.h)

    def layer_offsets(self, il: int) -> LayerOffsets:
        lo = LayerOffsets()
        if not lib().knj_model_layer_offsets(C.byref(self.cfg), il, C.byref(lo)):
            raise ValueError(f"layer {il} out of range")
        return lo

    def image_bytes(self) -> int:
        return lib().knj_model_image_bytes(self.h)

    def download_image(self) -> np.ndarray:
        n = self.image_bytes()
        out = np.empty(n, dtype=np.uint8)
        check(lib().knj_model_download_image(self.h, _ptr(out), n))
        return out

    def forward(self, tokens, want_logits: bool = True):
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        logits = np.empty(self.cfg.n_vocab, dtype=np.float32) if want_logits else None
        check(lib().knj_model_forward(self.h, _ptr(t), t.size,
                                      _ptr(logits) if logits is not None else None))
        return logits

    def decode_greedy(self, first: int, steps: int) -> np.ndarray:
        out = np.empty(steps, dtype=np.int32)
        check(lib().knj_model_decode_greedy(self.h, int(first), steps, _ptr(out)))
        return out

    def hidden(self, il: int) -> np.ndarray:
        out = np.empty(self.cfg.n_embd, dtype=np.float32)
        check(lib().knj_model_hidden(self.h, il, _ptr(out)))
        return out

    def topk(self, il: int):
        k = self.cfg.n_expert_used
        i = np.empty(k, dtype=np.int32)
        w = np.empty(k, dtype=np.float32)
        check(lib().knj_model_topk(self.h, il, _ptr(i), _ptr(w)))
        return i, w

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.n_vocab, dtype=np.float32)
        check(lib().knj_model_logits(self.h, _ptr(out)))
        return out

    def kv_shape(self):
        c = self.cfg
        return (c.n_layer, c.n_head_kv, c.n_ctx, c.head_dim)

    def kv_download(self):
        k = np.empty(self.kv_shape(), dtype=np.uint16)
        v = np.empty(self.kv_shape(), dtype=np.uint16)
        check(lib().knj_model_kv_download(self.h, _ptr(k), _ptr(v)))
        return k, v

    def kv_upload(self, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        check(lib().knj_model_kv_upload(self.h, _ptr(k), _ptr(v)))

    def time_decode(self, iters: int) -> float:
        ms = C.c_float()
        check(lib().knj_model_time_decode(self.h, iters, C.byref(ms)))
        return ms.value

    def profile(self, first: int, steps: int, cap: int = 4096):
        """Greedy decode with every launch timed (knj_model_profile): returns
        (tokens, spans as (name, layer, kernel, start_ns, end_ns), dropped)."""
        toks = np.zeros(steps, np.int32)
        sp = (Span * cap)()
        n = C.c_int(0)
        dropped = C.c_uint64(0)
        check(lib().knj_model_profile(self.h, first, steps, _ptr(toks), sp, cap, C.byref(n),
                                      C.byref(dropped)))
        spans = [(s.name.decode(), s.layer, s.kernel.decode(), s.start_ns, s.end_ns)
                 for s in sp[: n.value]]
        return toks, spans, dropped.value

    def transfer_bytes(self):
        h, d = C.c_uint64(0), C.c_uint64(0)
        check(lib().knj_model_transfer_bytes(self.h, C.byref(h), C.byref(d)))
        return h.value, d.value

    def time_experts(self, steps: int):
        """(gate/up, down) mean microseconds per launch over `steps` greedy decode
        steps launched directly, each expert launch recording HIP start/end events
        (n_layer * steps launches of each); advances the position by `steps`."""
        a, b = C.c_float(), C.c_float()
        check(lib().knj_model_time_experts(self.h, steps, C.byref(a), C.byref(b)))
        return a.value, b.value


class Batch:
    """n_seq sequences decoded in lockstep on a Model's weights (knj_batch_*);
    the model must stay open while the batch is used."""

    def __init__(self, model: "Model", n_seq: int, n_ctx: int):
        self.model = model
        self.cfg = model.cfg
        self.n_seq = n_seq
        self.n_ctx = n_ctx
        h = _P()
        check(lib().knj_batch_create(model.h, n_seq, n_ctx, C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().knj_batch_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self) -> int:
        return lib().knj_batch_pos(self.h)

    def forward(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(self.n_seq))
        out = np.empty((self.n_seq, self.cfg.n_vocab), dtype=np.float32)
        check(lib().knj_batch_forward(self.h, _ptr(t), _ptr(out)))
        return out

    def decode_greedy(self, first, steps: int) -> np.ndarray:
        f = np.ascontiguousarray(np.asarray(first, dtype=np.int32).reshape(self.n_seq))
        out = np.empty((steps, self.n_seq), dtype=np.int32)
        check(lib().knj_batch_decode_greedy(self.h, _ptr(f), steps, _ptr(out)))
        return out

    def fill_kv(self, n_pos: int, seed: int = 0) -> None:
        check(lib().knj_batch_fill_kv(self.h, n_pos, seed))

    def hidden(self, il: int, seq: int) -> np.ndarray:
        out = np.empty(self.cfg.n_embd, dtype=np.float32)
        check(lib().knj_batch_hidden(self.h, il, seq, _ptr(out)))
        return out

    def topk(self, il: int, seq: int):
        k = self.cfg.n_expert_used
        i = np.empty(k, dtype=np.int32)
        w = np.empty(k, dtype=np.float32)
        check(lib().knj_batch_topk(self.h, il, seq, _ptr(i), _ptr(w)))
        return i, w

    def kv_upload(self, seq: int, k: np.ndarray, v: np.ndarray) -> None:
        shape = (self.cfg.n_layer, self.cfg.n_head_kv, self.n_ctx, self.cfg.head_dim)
        k = np.ascontiguousarray(k, dtype=np.uint16).reshape(shape)
        v = np.ascontiguousarray(v, dtype=np.uint16).reshape(shape)
        check(lib().knj_batch_kv_upload(self.h, seq, _ptr(k), _ptr(v)))

    def set_pos(self, pos: int) -> None:
        check(lib().knj_batch_set_pos(self.h, pos))

    def kv_download(self, seq: int):
        shape = (self.cfg.n_layer, self.cfg.n_head_kv, self.n_ctx, self.cfg.head_dim)
        k = np.empty(shape, dtype=np.uint16)
        v = np.empty(shape, dtype=np.uint16)
        check(lib().knj_batch_kv_download(self.h, seq, _ptr(k), _ptr(v)))
        return k, v
