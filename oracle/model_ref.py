"""CPU restatement of the MiniCPM5 forward over the paged KV cache (numpy).

TEST INFRASTRUCTURE ONLY: the checker for the weight path (mc_model_load with
a model.wpk). Imported by tests/ only; the product library never calls it.

Restates native/runtime/forward.cpp:200-420 (the layer graph and its bf16
rounding points) with the reference kernels' arithmetic:
  * embedding row (embedding.cu:11-24);
  * RMSNorm: inv = 1/sqrt(mean(x^2) + eps) in fp32, out = bf16(x * inv * w)
    (rmsnorm.cu:95-125); residual add: res = bf16(res + x) before the norm
    (rmsnorm.cu:127-165);
  * projections y = bf16(x . W^T) with fp32 accumulation (gemm.cpp, gemv.cu);
  * RoPE + K/V append and attention through the KV oracle (kv_oracle.c:
    orc_rope_append mode 1, the kernel-exact fp32 statement; orc_attn_ref,
    the double softmax attention of kernel_ops.cpp:434-476);
  * SwiGLU: bf16(g / (1 + exp(-g)) * u) in fp32 (swiglu.cu:53-66);
  * logits bf16 of the last row, greedy argmax with ties to the lowest index
    (sampling.cu:69-100);
  * FP8 mode (precision MC_FP8, forward.cpp:117-130,444-456): single-token
    forwards run the four layer projections (and the lm_head when the
    package holds one) on e4m3 weights with fp32 row scales,
    y = bf16(scale[n] * sum_k e4m3(w[n][k]) x[k]) with fp32 accumulation
    (gemv_fp8.cu:3-7); e4m3 decodes by its bit layout (kernels.h:120-148:
    s.eeee.mmm, bias 7, subnormals m/8 * 2^-6, and S.1111.111 read as
    +-480 rather than NaN). Multi-token forwards stay bf16.
The vocabulary and the layer count are parameters (the hidden size, 2048, is
fixed by the 16 x 128 query heads) so that small instances can pin the
statement on the CPU.
"""
from __future__ import annotations

import numpy as np

from . import bf16_to_f32, f32_to_bf16, rope_append, attn_ref

HIDDEN, INTER, QKV = 2048, 6144, 2560
EPS = np.float32(1e-6)
THETA = 5.0e6


def bf16(x) -> np.ndarray:
    """fp32 -> nearest-even bf16 -> fp32."""
    return bf16_to_f32(f32_to_bf16(np.asarray(x, dtype=np.float32)))


def rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x [rows][n] (bf16 values as fp32), w [n] -> bf16(x * inv * w)."""
    x = np.asarray(x, dtype=np.float32)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(x.shape[-1]) + EPS)
    return bf16((x * inv) * w)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    return bf16(g / (np.float32(1.0) + np.exp(-g)) * u)


def e4m3_to_f32(q) -> np.ndarray:
    """e4m3 bit patterns (uint8) -> float32 by the bit layout: exponent field
    e (bias 7), mantissa m; e = 0 gives m/8 * 2^-6; S.1111.111 gives +-480."""
    q = np.asarray(q, dtype=np.uint8)
    e = ((q >> 3) & 0xF).astype(np.int32)
    m = (q & 0x7).astype(np.float64)
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7))
    return np.where(q & 0x80, -mag, mag).astype(np.float32)


def project_fp8(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """bf16(scale[n] * (x . e4m3(q)^T)[n]) with fp32 accumulation (the row
    scale applied after the sum)."""
    acc = np.asarray(x, np.float32) @ e4m3_to_f32(q).T
    return bf16(acc * np.asarray(scale, np.float32))


def project(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    """bf16(x . W^T) with fp32 operands (exact bf16 values) and fp32 BLAS
    accumulation."""
    return bf16(np.asarray(x, np.float32) @ np.asarray(W, np.float32).T)


class ModelRef:
    """Greedy decoder state for one session. `w` maps the wpk section names to
    fp32 arrays holding bf16 values ("embedding", "lm_head", "final_norm",
    "layer<i>.norm1|qkv|o|norm2|gate_up|down")."""

    def __init__(self, w: dict, layers: int, max_ctx: int = 256, P: int = 32, fp8=None):
        """fp8: None, or section name -> (e4m3 uint8 [N][K], fp32 scales [N])
        for the single-token projections (FP8 mode)."""
        self.w, self.layers, self.P, self.fp8 = w, layers, P, fp8
        self._dec = {}
        self.maxp = -(-max_ctx // P)
        self.pt = np.arange(self.maxp, dtype=np.uint32)
        self.pool = np.zeros(layers * self.maxp * P * 512, dtype=np.uint16)
        self.seq_len = 0
        self.next_token = None
        self.last_logits = None
        # when a dict: the last row of the residual at each layer's input and
        # after its two residual adds, and of the final norm's output, keyed
        # as the reference's debug dump files (debug_dump.h:5-12)
        self.capture = None

    def forward(self, ids) -> int:
        """Runs len(ids) tokens at positions seq_len.. and returns the greedy
        prediction after the last one (also kept as next_token)."""
        w, T, base = self.w, len(ids), self.seq_len
        if base + T > self.maxp * self.P:  # the C helpers write the pool unchecked
            raise ValueError(f"ModelRef: {base + T} tokens exceed max_ctx "
                             f"{self.maxp * self.P}")

        def proj(x, name):
            if T == 1 and self.fp8 is not None and name in self.fp8:
                q, scale = self.fp8[name]
                wq = self._dec.get(id(q))
                if wq is None:  # decoded once per code array (layer sets are shared)
                    wq = self._dec[id(q)] = e4m3_to_f32(q)
                return bf16((np.asarray(x, np.float32) @ wq.T) * np.asarray(scale, np.float32))
            return project(x, w[name])
        res = w["embedding"][np.asarray(ids)]
        normed = rmsnorm(res, w["layer0.norm1"])
        cap = self.capture
        for l in range(self.layers):
            p = f"layer{l}."
            if cap is not None:
                cap[p + "hidden_in"] = np.asarray(res[-1], np.float32).copy()
            qkv = f32_to_bf16(proj(normed, p + "qkv"))
            qkv = np.ascontiguousarray(qkv.reshape(T, QKV))
            rope_append(qkv, T, base, l, self.pt, self.P, self.maxp, THETA, 1, self.pool)
            att = bf16_to_f32(attn_ref(qkv, T, base, l, self.pool, self.pt, self.P, self.maxp))
            o = proj(att, p + "o")
            res = bf16(res + o)
            if cap is not None:
                cap[p + "attn_out"] = np.asarray(res[-1], np.float32).copy()
            normed = rmsnorm(res, w[p + "norm2"])
            gu = proj(normed, p + "gate_up")
            mlp = silu_mul(gu[:, :INTER], gu[:, INTER:])
            d = proj(mlp, p + "down")
            res = bf16(res + d)
            if cap is not None:
                cap[p + "mlp_out"] = np.asarray(res[-1], np.float32).copy()
            nxt = w[f"layer{l + 1}.norm1"] if l + 1 < self.layers else w["final_norm"]
            normed = rmsnorm(res, nxt)
        if cap is not None:
            cap["final_hidden"] = np.asarray(normed[-1], np.float32).copy()
        logits = proj(normed[-1:], "lm_head")[0]
        self.seq_len += T
        self.last_logits = logits
        self.next_token = int(np.argmax(logits))  # first index of the maximum
        return self.next_token

    def decode(self) -> int:
        """The reference's decode step (decode_executor.cpp:171-230): returns
        the pending prediction and runs the forward on it."""
        emitted = self.next_token
        self.forward([emitted])
        return emitted
