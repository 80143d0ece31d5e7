"""Writes model_forward_small.json: the logits of the reference's whole-model
numpy statement (tools/reference_forward.py: MiniCPM5Ref.forward :254-302,
lm_head :304-326, greedy :328-333, with its bf16 kernels :158-242) for a
2-layer model with a 512-token vocabulary and random weights
(wpk_util.golden_small_model(seed=2024)): a 6-token prefill, then 5 greedy
decode steps, each feeding the previous prediction back as the reference's
golden generator does (:349-400); then the same in FP8 mode
(use_fp8=True for the single-token steps, :254-266,304-326): the four layer
projections and the lm_head quantized per row by wpk_util.quantize_rows
(e4m3 codes + fp32 row scales, the layout of model_fp8.wpk).

Run in the build container (it imports the reference from /root/reference;
the GPU box has no copy): python tests/golden/make_model_forward_golden.py
The reference module's layer count and vocabulary are module constants; the
script sets them to the small model's, and hands the forward a weight store
holding the generated arrays (the reference's WeightStore reads them from a
full-size package).
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import wpk_util as W  # noqa: E402

SEED, VOCAB, LAYERS = 2024, 512, 2
PROMPT = [5, 300, 17, 511, 0, 42]
STEPS = 5


class Store:
    def __init__(self, w):
        self.w = w

    def matrix(self, name):
        return self.w[name]

    def vector(self, name):
        return self.w[name]

    def matrix_fp8(self, name):
        return self.q[name]


def main():
    sys.path.insert(0, "/root/reference/tools")
    import reference_forward as rf
    rf.NUM_LAYERS, rf.VOCAB = LAYERS, VOCAB
    w = W.golden_small_model(SEED, VOCAB, LAYERS)
    store = Store(w)
    store.q = W.golden_small_fp8(w, LAYERS)
    model = rf.MiniCPM5Ref(store)

    def generate(fp8):
        cap = len(PROMPT) + STEPS + 1
        kv_k = [np.zeros((cap, 256), dtype=np.uint16) for _ in range(LAYERS)]
        kv_v = [np.zeros((cap, 256), dtype=np.uint16) for _ in range(LAYERS)]
        logits, _, _ = model.forward(PROMPT, kv_k, kv_v, kv_len=0, pos_start=0)
        out_logits, tokens = [logits.tolist()], [model.greedy(logits)]
        n = len(PROMPT)
        for _ in range(STEPS):
            logits, _, _ = model.forward([tokens[-1]], kv_k, kv_v, kv_len=n, pos_start=n,
                                         use_fp8=fp8)
            n += 1
            out_logits.append(logits.tolist())
            tokens.append(model.greedy(logits))
        return tokens, out_logits

    tokens, out_logits = generate(False)
    tokens8, out_logits8 = generate(True)
    doc = {"source": "tools/reference_forward.py MiniCPM5Ref (numpy, bf16 storage, fp32 math)",
           "weights": "tests/wpk_util.py golden_small_model(seed, vocab, layers); FP8: "
                      "golden_small_fp8 (quantize_rows of the same weights)",
           "seed": SEED, "vocab": VOCAB, "layers": LAYERS, "prompt": PROMPT,
           "tokens": tokens, "logits_bf16": out_logits,
           "fp8": {"tokens": tokens8, "logits_bf16": out_logits8}}
    with open(os.path.join(HERE, "model_forward_small.json"), "w") as f:
        json.dump(doc, f, separators=(",", ":"))
    print("tokens", tokens, "fp8", tokens8)


if __name__ == "__main__":
    main()
