"""A minimal GGUF v2/v3 writer (test infrastructure): writes metadata and
tensors so the library's parser and loader can be checked on files whose
contents are known.

Layout written: b"GGUF", u32 version, u64 n_tensors, u64 n_kv; each KV as
(string key, u32 type, value); each tensor record as (string name, u32
n_dims, u64 dims..., u32 ggml type, u64 offset); zero padding to the
alignment; then each tensor's bytes at its offset (offsets aligned).
Strings are u64 length + UTF-8 bytes; arrays are u32 element type + u64
count + elements.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}

GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 8, 12, 14


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, it) for it in items)
    return struct.pack(_FMT[vtype], v)


def write_gguf(path: str, kvs: list, tensors: list, version: int = 3, alignment: int | None = None) -> dict:
    """kvs: [(key, vtype, value)]; tensors: [(name, ggml_type, dims, bytes)]
    with dims innermost first.  general.alignment is added when `alignment`
    is given.  Returns {name: (offset, size)} and the data section offset."""
    align = alignment or 32
    kv_list = list(kvs)
    if alignment is not None:
        kv_list.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv_list))
    body = b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kv_list)
    offsets, off = {}, 0
    recs = []
    for name, gtype, dims, data in tensors:
        off = (off + align - 1) // align * align
        offsets[name] = (off, len(data))
        recs.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) +
                    struct.pack("<IQ", gtype, off))
        off += len(data)
    meta = head + body + b"".join(recs)
    data_off = (len(meta) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(meta)
        f.write(b"\0" * (data_off - len(meta)))
        pos = 0
        for name, _, _, data in tensors:
            o, _ = offsets[name]
            f.write(b"\0" * (o - pos))
            f.write(bytes(data))
            pos = o + len(data)
    return {"offsets": offsets, "data_offset": data_off}


def moe_layer_tensors(layer: int, H: int, I: int, Ish: int, E: int, seed: int, with_shgate=True, with_norm=True,
                      types=None):
    """The MoE tensors of block `layer` (names of loader.c:162-164,
    :559-569 and one_layer.cu:964-975, :1413), synthetic values.  types:
    ggml types of gate, up, down, gate_shexp, up_shexp, down_shexp (each
    Q4_K or Q6_K; default Q4_K, Q4_K, Q6_K for both)."""
    from breadv2_amd import synth

    tg, tu, td, tgs, tus, tds = types or (GGML_Q4_K, GGML_Q4_K, GGML_Q6_K, GGML_Q4_K, GGML_Q4_K, GGML_Q6_K)

    def q(qtype, n_blocks, sd):
        return synth.synth_q4k(n_blocks, sd) if qtype == GGML_Q4_K else synth.synth_q6k(n_blocks, sd)

    rng = np.random.default_rng(seed)
    t = [
        (f"blk.{layer}.ffn_gate_exps.weight", tg, [H, I, E], q(tg, E * I * H // 256, seed + 1)),
        (f"blk.{layer}.ffn_up_exps.weight", tu, [H, I, E], q(tu, E * I * H // 256, seed + 2)),
        (f"blk.{layer}.ffn_down_exps.weight", td, [I, H, E], q(td, E * H * I // 256, seed + 3)),
        (f"blk.{layer}.ffn_gate_shexp.weight", tgs, [H, Ish], q(tgs, Ish * H // 256, seed + 4)),
        (f"blk.{layer}.ffn_up_shexp.weight", tus, [H, Ish], q(tus, Ish * H // 256, seed + 5)),
        (f"blk.{layer}.ffn_down_shexp.weight", tds, [Ish, H], q(tds, H * Ish // 256, seed + 6)),
        (f"blk.{layer}.ffn_gate_inp.weight", GGML_F32, [H, E],
         (0.02 * rng.standard_normal(E * H)).astype(np.float32).view(np.uint8)),
    ]
    if with_shgate:
        t.append((f"blk.{layer}.ffn_gate_inp_shexp.weight", GGML_F16, [H],
                  (0.02 * rng.standard_normal(H)).astype(np.float16).view(np.uint8)))
    if with_norm:
        t.append((f"blk.{layer}.post_attention_norm.weight", GGML_F32, [H],
                  (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32).view(np.uint8)))
    return t
