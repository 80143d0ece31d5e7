"""GPU tests of the process-wide switches the reference reads once from the
environment, each case in a child process of its own:

* MC_ROPE_TABLE_OFF (native/runtime/forward.cpp:248-262): the RoPE kernel
  computes its frequencies instead of reading the table, and a decode step
  runs it before the attention instead of the attention's phase0 append.
  Same values bit for bit, so the logits equal the default run's.
* MC_ATTN_CHUNK512_ON (native/kernels/sm120/kernels.h:292-304): a session
  of more than 114688 positions decodes with 512-position chunks; its logits
  are checked against the forward oracle.
* MC_PREFILL_CHUNK (native/runtime/prefill_executor.cpp:27-50): tokens per
  prefill forward, 8448..65535; a prompt is prefilled in chunks of that
  size (bit-identical to mc_prefill calls of the chunk lengths), and an
  invalid value keeps 8448 with a warning.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import wpk_util as W

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PROMPT = [1, 500, 130559, 77, 9, 12345, 3, 3, 42]

# child: prefill PROMPT, 3 greedy decodes; writes tokens, chunk size and the
# logits after each step
CHILD = r"""
import importlib, json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
rt = importlib.import_module("minicpm5-5080fast_amd.runtime")
path, ctx, graphs, out = sys.argv[2], int(sys.argv[3]), int(sys.argv[4]), sys.argv[5]
m = rt.Model(path, rt.model_options(max_context_tokens=ctx, max_sessions=1,
                                    enable_cuda_graph=graphs))
s = rt.Session(m)
s.prefill(json.loads(sys.argv[6]))
logits, toks = [s.last_logits()], []
cfg = rt.gen_config(max_new_tokens=8)
for _ in range(3):
    toks.append(s.decode_one(cfg))
    logits.append(s.last_logits())
np.save(out, np.stack(logits))
print(json.dumps({"tokens": toks, "chunk": s.attn_chunk()}))
s.close()
m.close()
"""


SWITCHES = ("MC_ROPE_TABLE_OFF", "MC_ATTN_CHUNK512_ON", "MC_ATTN_CHUNK512_OFF",
            "MC_PREFILL_CHUNK")


def run_child(path, ctx, graphs, tmp_path, name, env):
    e = {k: v for k, v in os.environ.items() if k not in SWITCHES}
    e.update(env)
    out = str(tmp_path / (name + ".npy"))
    print("child", name, env, ctx, graphs, flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT, path, str(ctx), str(graphs), out,
                        json.dumps(PROMPT)], env=e, capture_output=True, text=True,
                       timeout=100)
    assert r.returncode == 0, r.stderr[-2000:]
    info = json.loads(r.stdout.strip().splitlines()[-1])
    return info, np.load(out)


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("wpk_env")
    secs = W.model_sections(2)
    blobs = W.random_blobs(4321, 2, scale=1.0)
    W.write_wpk(os.path.join(d, "model.wpk"), secs, blobs)
    return str(d), W.weights_f32(secs, blobs)


def test_rope_table_off_equals_default(model_dir, tmp_path):
    path, _ = model_dir
    base_info, base = run_child(path, 4096, 0, tmp_path, "base", {})
    for graphs in (0, 1):
        info, got = run_child(path, 4096, graphs, tmp_path, "off%d" % graphs,
                              {"MC_ROPE_TABLE_OFF": "1"})
        assert info["tokens"] == base_info["tokens"]
        assert np.array_equal(got, base), graphs


def test_chunk512_session_vs_oracle(model_dir, tmp_path):
    from oracle import model_ref as R
    path, w = model_dir
    info, got = run_child(path, 131072, 1, tmp_path, "c512", {"MC_ATTN_CHUNK512_ON": "1"})
    assert info["chunk"] == 512
    d_info, _ = run_child(path, 131072, 1, tmp_path, "c256", {})
    assert d_info["chunk"] == 256
    ref = R.ModelRef(w, 42)
    ref.forward(PROMPT)
    for step in range(4):
        ref_l = ref.last_logits
        diff = got[step].astype(np.float64) - ref_l.astype(np.float64)
        rel = np.linalg.norm(diff) / np.linalg.norm(ref_l)
        cos = float(got[step] @ ref_l / (np.linalg.norm(got[step]) * np.linalg.norm(ref_l)))
        print("step", step, "rel", rel, "cos", cos)
        assert rel < 2e-2 and cos > 0.999
        if step < 3:
            ref.next_token = info["tokens"][step]
            ref.decode()


# child: one 9552-token prompt prefilled whole and as two mc_prefill calls
# split at 9000 and at 8448; prints which splits equal the whole bit for bit
CHILD_PF = r"""
import importlib, json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
rt = importlib.import_module("minicpm5-5080fast_amd.runtime")
m = rt.Model(sys.argv[2], rt.model_options(max_context_tokens=16384, max_sessions=3))
prompt = [(i * 7919 + 11) % 130560 for i in range(9552)]
whole = rt.Session(m)
whole.prefill(prompt)
res = {}
for cut in (9000, 8448):
    s = rt.Session(m)
    s.prefill(prompt[:cut])
    s.prefill(prompt[cut:])
    res[str(cut)] = bool(np.array_equal(whole.last_logits(), s.last_logits()))
    s.close()
whole.close()
m.close()
print(json.dumps(res))
"""


@pytest.mark.parametrize("value,cut", [("9000", "9000"), (None, "8448"), ("100", "8448")])
def test_prefill_chunk_from_environment(model_dir, value, cut):
    path, _ = model_dir
    e = {k: v for k, v in os.environ.items() if k not in SWITCHES}
    if value is not None:
        e["MC_PREFILL_CHUNK"] = value
    print("child prefill chunk", value, flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD_PF, ROOT, path], env=e,
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr[-2000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res[cut], res
    assert ("MC_PREFILL_CHUNK" in r.stderr) == (value == "100")
