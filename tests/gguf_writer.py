"""A minimal GGUF (version 3) writer for tests: metadata scalars and tensors.

Layout written from the GGUF container format: magic "GGUF", version, tensor
count, metadata count; each metadata entry as (string key, u32 value type,
value); each tensor info as (string name, u32 n_dims, u64 dims with dims[0]
fastest, u32 ggml type, u64 offset into the data section); the data section
from the next multiple of 32, each tensor 32-byte aligned.
"""
import struct

import numpy as np

U32, I32, F32, STRING, U64 = 4, 5, 6, 8, 10
ALIGN = 32


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == U32:
        return struct.pack("<I", v)
    if vtype == I32:
        return struct.pack("<i", v)
    if vtype == F32:
        return struct.pack("<f", v)
    if vtype == U64:
        return struct.pack("<Q", v)
    if vtype == STRING:
        return _str(v)
    raise ValueError(vtype)


def write_gguf(path, meta, tensors):
    """meta: [(key, vtype, value)]; tensors: [(name, dims, ggml_type, bytes)]."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta))
    for key, vtype, v in meta:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += (len(data) + ALIGN - 1) // ALIGN * ALIGN
    for (name, dims, gtype, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gtype, o)
    pad = (-len(head)) % ALIGN
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (_, _, _, data), o in zip(tensors, offsets):
            data = bytes(np.ascontiguousarray(data).view(np.uint8).reshape(-1))
            f.write(data + b"\0" * ((-len(data)) % ALIGN))


def qwen3moe_meta(cfg: dict, ctx_train: int = 40960):
    p = "qwen3moe."
    return [("general.architecture", STRING, "qwen3moe"),
            (p + "block_count", U32, cfg["n_layer"]),
            (p + "embedding_length", U32, cfg["n_embd"]),
            (p + "attention.head_count", U32, cfg["n_head"]),
            (p + "attention.head_count_kv", U32, cfg["n_head_kv"]),
            (p + "attention.key_length", U32, cfg["head_dim"]),
            (p + "expert_feed_forward_length", U32, cfg["n_ff"]),
            (p + "expert_count", U32, cfg["n_expert"]),
            (p + "expert_used_count", U32, cfg["n_expert_used"]),
            (p + "context_length", U32, ctx_train),
            (p + "attention.layer_norm_rms_epsilon", F32, cfg.get("rms_eps", 1e-6)),
            (p + "rope.freq_base", F32, cfg.get("rope_base", 1e6))]


def _align256(v: int) -> int:
    return (v + 255) // 256 * 256


def tensors_from_image(cfg, image):
    """The GGUF tensors of a weight image in this build's layout
    (include/knj_model.h), wqkv split back into attn_q/attn_k/attn_v."""
    import ctypes as C

    import kanjoos_amd as K

    c = cfg if isinstance(cfg, K.ModelConfig) else K.ModelConfig(**cfg)
    H, F, E, V = c.n_embd, c.n_ff, c.n_expert, c.n_vocab
    QD, KVD, D = c.n_head * c.head_dim, c.n_head_kv * c.head_dim, c.head_dim
    rb = K.row_bytes
    img = np.asarray(image, dtype=np.uint8)

    def lo(il):
        o = K.LayerOffsets()
        assert K.lib().knj_model_layer_offsets(C.byref(c), il, C.byref(o))
        return o

    out = [("token_embd.weight", [H, V], c.type_embd, img[0:rb(c.type_embd, H) * V])]
    for il in range(c.n_layer):
        o = lo(il)
        b = f"blk.{il}."
        ra = rb(c.type_attn, H)
        out += [(b + "attn_norm.weight", [H], 0, img[o.attn_norm:o.attn_norm + 4 * H]),
                (b + "ffn_norm.weight", [H], 0, img[o.ffn_norm:o.ffn_norm + 4 * H]),
                (b + "attn_q_norm.weight", [D], 0, img[o.q_norm:o.q_norm + 4 * D]),
                (b + "attn_k_norm.weight", [D], 0, img[o.k_norm:o.k_norm + 4 * D]),
                (b + "attn_q.weight", [H, QD], c.type_attn, img[o.wqkv:o.wqkv + ra * QD]),
                (b + "attn_k.weight", [H, KVD], c.type_attn,
                 img[o.wqkv + ra * QD:o.wqkv + ra * (QD + KVD)]),
                (b + "attn_v.weight", [H, KVD], c.type_attn,
                 img[o.wqkv + ra * (QD + KVD):o.wqkv + ra * (QD + 2 * KVD)]),
                (b + "attn_output.weight", [QD, H], c.type_attn,
                 img[o.wo:o.wo + rb(c.type_attn, QD) * H]),
                (b + "ffn_gate_inp.weight", [H, E], 0, img[o.router:o.router + 4 * H * E]),
                (b + "ffn_gate_exps.weight", [H, F, E], c.type_gate_up,
                 img[o.gate:o.gate + rb(c.type_gate_up, H) * F * E]),
                (b + "ffn_up_exps.weight", [H, F, E], c.type_gate_up,
                 img[o.up:o.up + rb(c.type_gate_up, H) * F * E]),
                (b + "ffn_down_exps.weight", [F, H, E], c.type_down,
                 img[o.down:o.down + rb(c.type_down, F) * H * E])]
    last = lo(c.n_layer - 1)
    onorm = _align256(last.down + rb(c.type_down, F) * H * E)
    head = _align256(onorm + 4 * H)
    out += [("output_norm.weight", [H], 0, img[onorm:onorm + 4 * H]),
            ("output.weight", [H, V], c.type_head, img[head:head + rb(c.type_head, H) * V])]
    return out
