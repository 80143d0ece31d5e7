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


# ---- FP8 package (model_fp8.wpk) ----
# The reference's FP8 mode reads a second package, model_fp8.wpk, holding the
# 42 x {qkv, o, gate_up, down} projections (and optionally the lm_head) as
# dtype-2 sections: e4m3 bytes [N][K] plus fp32 per-row scales at the entry's
# scale_offset / scale_bytes (weight_loader.cpp:465-620).

def _e4m3_values():
    """Values of the non-negative finite codes 0x00..0x7E (ascending)."""
    codes = np.arange(0x7F, dtype=np.int64)
    e, m = codes >> 3, (codes & 7).astype(np.float64)
    return np.where(e == 0, m / 8 * 2.0 ** -6, (1 + m / 8) * np.exp2(e - 7))


_E4M3_POS = _e4m3_values()


def f32_to_e4m3(x) -> np.ndarray:
    """fp32 -> e4m3 codes: the nearest value among the 127 non-negative
    finite codes (ties to the even code), magnitudes past 448 saturating to
    448 (0x7E), sign in bit 7."""
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), 448.0)
    hi = np.clip(np.searchsorted(_E4M3_POS, a), 1, 0x7E)
    lo = hi - 1
    dl, dh = a - _E4M3_POS[lo], _E4M3_POS[hi] - a
    pick_hi = (dh < dl) | ((dh == dl) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)


def quantize_rows(w_bf16) -> tuple:
    """Per-row e4m3 quantization of a bf16 [N][K] matrix: scale[n] =
    max|row| / 448 (at least 1e-12), codes = e4m3(w / scale)."""
    w = (np.asarray(w_bf16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    scale = np.maximum(np.max(np.abs(w), axis=-1) / np.float32(448.0),
                       np.float32(1e-12)).astype(np.float32)
    return f32_to_e4m3(w / scale[:, None]), scale


def fp8_sections(layer_sets: int = 2, lm_head: bool = True):
    """[(name, (N, K), blob key)] of model_fp8.wpk; layer i uses set i % sets."""
    out = []
    for i in range(LAYERS):
        k = i % layer_sets
        out += [(f"layer{i}.qkv", (QKV, HIDDEN), f"qkv.{k}"),
                (f"layer{i}.o", (HIDDEN, HIDDEN), f"o.{k}"),
                (f"layer{i}.gate_up", (2 * INTER, HIDDEN), f"gate_up.{k}"),
                (f"layer{i}.down", (HIDDEN, INTER), f"down.{k}")]
    if lm_head:
        out.append(("lm_head", (VOCAB, HIDDEN), "table"))
    return out


def fp8_blobs(bf16_blobs, layer_sets: int = 2, lm_head: bool = True):
    """Quantized blobs key -> (codes uint8 [N][K], scales fp32 [N]) of the
    bf16 blobs of random_blobs / model_sections."""
    keys = [f"{n}.{k}" for k in range(layer_sets) for n in ("qkv", "o", "gate_up", "down")]
    if lm_head:
        keys.append("table")
    return {key: quantize_rows(bf16_blobs[key]) for key in keys}


def write_fp8_wpk(path, sections, blobs, entry_patch=None):
    """sections: [(name, (N, K), key)]; blobs: key -> (codes, scales) or
    (data bytes, scale bytes) ints for holes. Data areas are 256-byte aligned,
    each blob's scales follow its codes."""
    hdr_bytes = 64 + len(sections) * 132
    cursor = (hdr_bytes + 255) // 256 * 256
    data_start = cursor
    place = {}
    for _, _, key in sections:
        if key in place:
            continue
        b = blobs[key]
        nd, ns = (b[0], b[1]) if isinstance(b[0], int) else (b[0].nbytes, b[1].nbytes)
        place[key] = (cursor, cursor + (nd + 255) // 256 * 256)
        cursor = place[key][1] + (ns + 255) // 256 * 256
    with open(path, "wb") as f:
        f.write(struct.pack("<IHH32sIIQQ", MAGIC, ABI, TARGET_SM, b"\x00" * 32, len(sections),
                            0, 64, data_start))
        for i, (name, (n, k), key) in enumerate(sections):
            d = {"hash": fnv1a64(name), "dtype": 2, "layout": 0, "rank": 2,
                 "dims": [n, k] + [0] * 6, "offset": place[key][0], "bytes": n * k,
                 "scale_offset": place[key][1], "scale_bytes": n * 4}
            if entry_patch is not None:
                entry_patch(i, d)
            f.write(struct.pack("<QIII8IQQQQ6Q", d["hash"], d["dtype"], d["layout"], d["rank"],
                                *d["dims"], d["offset"], d["bytes"], d["scale_offset"],
                                d["scale_bytes"], *([0] * 6)))
        for key, (do, so) in place.items():
            b = blobs[key]
            if isinstance(b[0], int):
                continue
            f.seek(do)
            f.write(np.ascontiguousarray(b[0], dtype=np.uint8).tobytes())
            f.seek(so)
            f.write(np.ascontiguousarray(b[1], dtype=np.float32).tobytes())
        f.truncate(cursor)
    return cursor


def fp8_weights(sections, blobs):
    """Section name -> (codes, scales) for oracle/model_ref.ModelRef(fp8=...)."""
    return {name: blobs[key] for name, _, key in sections}


def golden_small_fp8(w, layers: int):
    """FP8 copies (codes, scales) of the projections and the lm_head of a
    golden_small_model weight dict."""
    names = ["lm_head"] + [f"layer{i}.{n}" for i in range(layers)
                           for n in ("qkv", "o", "gate_up", "down")]
    return {n: quantize_rows(w[n]) for n in names}


def fp8_sparse_blobs(layer_sets: int = 2):
    """(code bytes, scale bytes) of every fp8_sections blob (a file of holes)."""
    b = {"table": (VOCAB * HIDDEN, VOCAB * 4)}
    for k in range(layer_sets):
        b.update({f"qkv.{k}": (QKV * HIDDEN, QKV * 4), f"o.{k}": (HIDDEN * HIDDEN, HIDDEN * 4),
                  f"gate_up.{k}": (2 * INTER * HIDDEN, 2 * INTER * 4),
                  f"down.{k}": (HIDDEN * INTER, HIDDEN * 4)})
    return b


def fp8_arena_bytes(sections) -> int:
    """Device bytes of the FP8 copies: codes then scales of each section,
    each 256-byte aligned, in the loader's order (layers, then lm_head)."""
    c = 0
    for _, (n, k), _ in sections:
        c = (c + n * k + 255) // 256 * 256
        c = (c + n * 4 + 255) // 256 * 256
    return c
