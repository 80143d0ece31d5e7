"""Writes model.wpk weight packages for the tests (the reference's WPK v1
layout, native/runtime/weight_loader.h:4-10): a 64-byte header, 132-byte TOC
entries keyed by the FNV-1a 64 hash of the section name, then the data.

Sections may share one data blob (the package format allows any offsets), so
a full-geometry model (42 layers, vocabulary 130560) fits in a few hundred
MB: the tests give the even and odd layers two weight sets and let
"embedding" and "lm_head" share one table. Blobs given as an int are byte
counts left as a hole (a sparse file: the loader's checks do not read data).
"""
from __future__ import annotations

import struct

import numpy as np

HIDDEN, INTER, QKV, VOCAB, LAYERS = 2048, 6144, 2560, 130560, 42
MAGIC, ABI, TARGET_SM = 0x31504B4D, 2, 120


def fnv1a64(name: str) -> int:
    h = 14695981039346656037
    for c in name.encode():
        h ^= c
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def model_sections(layer_sets: int = 2):
    """[(name, dims, blob key)] of the full model; layer i uses weight set
    i % layer_sets."""
    out = [("embedding", (VOCAB, HIDDEN), "table"), ("lm_head", (VOCAB, HIDDEN), "table"),
           ("final_norm", (HIDDEN,), "final_norm")]
    for i in range(LAYERS):
        k = i % layer_sets
        out += [(f"layer{i}.norm1", (HIDDEN,), f"norm1.{k}"),
                (f"layer{i}.qkv", (QKV, HIDDEN), f"qkv.{k}"),
                (f"layer{i}.o", (HIDDEN, HIDDEN), f"o.{k}"),
                (f"layer{i}.norm2", (HIDDEN,), f"norm2.{k}"),
                (f"layer{i}.gate_up", (2 * INTER, HIDDEN), f"gate_up.{k}"),
                (f"layer{i}.down", (HIDDEN, INTER), f"down.{k}")]
    return out


def write_wpk(path, sections, blobs, header=None, entry_patch=None):
    """sections: [(name, dims, blob key)]; blobs: key -> uint16 array or byte
    count (hole). header: overrides of the header fields; entry_patch(i, d)
    may edit entry i's field dict before it is packed."""
    hdr = {"magic": MAGIC, "abi": ABI, "target_sm": TARGET_SM, "count": len(sections),
           "reserved": 0, "toc_offset": 64}
    hdr.update(header or {})
    toc_bytes = len(sections) * 132
    data_start = (64 + toc_bytes + 255) // 256 * 256
    hdr.setdefault("data_start", data_start)
    offsets, cursor = {}, data_start
    keys = list(dict.fromkeys(k for _, _, k in sections))
    for k in keys:
        b = blobs[k]
        n = b if isinstance(b, int) else b.nbytes
        offsets[k] = cursor
        cursor += (n + 255) // 256 * 256
    with open(path, "wb") as f:
        f.write(struct.pack("<IHH32sIIQQ", hdr["magic"], hdr["abi"], hdr["target_sm"],
                            b"\x00" * 32, hdr["count"], hdr["reserved"], hdr["toc_offset"],
                            hdr["data_start"]))
        for i, (name, dims, k) in enumerate(sections):
            n = int(np.prod(dims)) * 2
            d = {"hash": fnv1a64(name), "dtype": 0, "layout": 0, "rank": len(dims),
                 "dims": list(dims) + [0] * (8 - len(dims)), "offset": offsets[k], "bytes": n}
            if entry_patch is not None:
                entry_patch(i, d)
            f.write(struct.pack("<QIII8IQQQQ6Q", d["hash"], d["dtype"], d["layout"], d["rank"],
                                *d["dims"], d["offset"], d["bytes"], 0, 0, *([0] * 6)))
        for k in keys:
            b = blobs[k]
            if isinstance(b, int):
                continue
            f.seek(offsets[k])
            f.write(np.ascontiguousarray(b, dtype=np.uint16).tobytes())
        f.truncate(cursor)
    return cursor


def sparse_blobs(layer_sets: int = 2):
    """Byte counts of every blob of model_sections (a file of holes)."""
    sizes = {"table": VOCAB * HIDDEN * 2, "final_norm": HIDDEN * 2}
    for k in range(layer_sets):
        sizes.update({f"norm1.{k}": HIDDEN * 2, f"qkv.{k}": QKV * HIDDEN * 2,
                      f"o.{k}": HIDDEN * HIDDEN * 2, f"norm2.{k}": HIDDEN * 2,
                      f"gate_up.{k}": 2 * INTER * HIDDEN * 2, f"down.{k}": HIDDEN * INTER * 2})
    return sizes


def arena_bytes(sections) -> int:
    """Device bytes the loader places the sections in (256-byte aligned, in
    the model's section order)."""
    c = 0
    for _, dims, _ in sections:
        c = (c + 255) // 256 * 256 + int(np.prod(dims)) * 2
    return c


def f32_to_bf16(x) -> np.ndarray:
    """Nearest-even fp32 -> bf16 bits (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)) \
        .astype(np.uint16)


def random_blobs(seed: int, layer_sets: int = 2, scale: float = 1.0):
    """bf16 weight blobs (uint16) of a random model: embedding rows ~N(0, 1),
    projections ~N(0, 1/fan_in) * scale, norms ~1 + N(0, 0.1)."""
    rng = np.random.default_rng(seed)

    def mat(rows, cols, s):
        return f32_to_bf16(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(s))

    def norm():
        return f32_to_bf16(1.0 + 0.1 * rng.standard_normal(HIDDEN, dtype=np.float32))

    b = {"table": mat(VOCAB, HIDDEN, 1.0), "final_norm": norm()}
    for k in range(layer_sets):
        b[f"norm1.{k}"] = norm()
        b[f"qkv.{k}"] = mat(QKV, HIDDEN, scale / HIDDEN ** 0.5)
        b[f"o.{k}"] = mat(HIDDEN, HIDDEN, scale / HIDDEN ** 0.5)
        b[f"norm2.{k}"] = norm()
        b[f"gate_up.{k}"] = mat(2 * INTER, HIDDEN, scale / HIDDEN ** 0.5)
        b[f"down.{k}"] = mat(HIDDEN, INTER, scale / INTER ** 0.5)
    return b


def weights_f32(sections, blobs):
    """Section name -> fp32 array (shared blobs are shared arrays)."""
    def bf16_to_f32(b):
        return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    cache = {}
    out = {}
    for name, dims, k in sections:
        if k not in cache:
            cache[k] = bf16_to_f32(blobs[k]).reshape(dims)
        out[name] = cache[k]
    return out


def golden_small_model(seed: int, vocab: int, layers: int):
    """bf16 weights (uint16) of a small-vocabulary model of the full layer
    shapes, generated from `seed` in a fixed order (the model-forward golden
    fixture is made from these): embedding ~N(0, 1), projections
    ~N(0, 1/fan_in), norms ~1 + N(0, 0.1)."""
    rng = np.random.default_rng(seed)

    def mat(rows, cols):
        return f32_to_bf16(rng.standard_normal((rows, cols), dtype=np.float32)
                           * np.float32(cols ** -0.5))

    def norm():
        return f32_to_bf16(1.0 + 0.1 * rng.standard_normal(HIDDEN, dtype=np.float32))

    w = {"embedding": f32_to_bf16(rng.standard_normal((vocab, HIDDEN), dtype=np.float32)),
         "lm_head": mat(vocab, HIDDEN), "final_norm": norm()}
    for i in range(layers):
        p = f"layer{i}."
        w[p + "norm1"], w[p + "norm2"] = norm(), norm()
        w[p + "qkv"] = mat(QKV, HIDDEN)
        w[p + "o"] = mat(HIDDEN, HIDDEN)
        w[p + "gate_up"] = mat(2 * INTER, HIDDEN)
        w[p + "down"] = mat(HIDDEN, INTER)
    return w
