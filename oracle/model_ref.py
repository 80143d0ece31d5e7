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
    (sampling.cu:69-100).
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


def project(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    """bf16(x . W^T) with fp32 operands (exact bf16 values) and fp32 BLAS
    accumulation."""
    return bf16(np.asarray(x, np.float32) @ np.asarray(W, np.float32).T)


class ModelRef:
    """Greedy decoder state for one session. `w` maps the wpk section names to
    fp32 arrays holding bf16 values ("embedding", "lm_head", "final_norm",
    "layer<i>.norm1|qkv|o|norm2|gate_up|down")."""

    def __init__(self, w: dict, layers: int, max_ctx: int = 256, P: int = 32):
        self.w, self.layers, self.P = w, layers, P
        self.maxp = -(-max_ctx // P)
        self.pt = np.arange(self.maxp, dtype=np.uint32)
        self.pool = np.zeros(layers * self.maxp * P * 512, dtype=np.uint16)
        self.seq_len = 0
        self.next_token = None
        self.last_logits = None

    def forward(self, ids) -> int:
        """Runs len(ids) tokens at positions seq_len.. and returns the greedy
        prediction after the last one (also kept as next_token)."""
        w, T, base = self.w, len(ids), self.seq_len
        res = w["embedding"][np.asarray(ids)]
        normed = rmsnorm(res, w["layer0.norm1"])
        for l in range(self.layers):
            p = f"layer{l}."
            qkv = f32_to_bf16(project(normed, w[p + "qkv"]))
            qkv = np.ascontiguousarray(qkv.reshape(T, QKV))
            rope_append(qkv, T, base, l, self.pt, self.P, self.maxp, THETA, 1, self.pool)
            att = bf16_to_f32(attn_ref(qkv, T, base, l, self.pool, self.pt, self.P, self.maxp))
            o = project(att, w[p + "o"])
            res = bf16(res + o)
            normed = rmsnorm(res, w[p + "norm2"])
            gu = project(normed, w[p + "gate_up"])
            mlp = silu_mul(gu[:, :INTER], gu[:, INTER:])
            d = project(mlp, w[p + "down"])
            res = bf16(res + d)
            nxt = w[f"layer{l + 1}.norm1"] if l + 1 < self.layers else w["final_norm"]
            normed = rmsnorm(res, nxt)
        logits = project(normed[-1:], w["lm_head"])[0]
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
