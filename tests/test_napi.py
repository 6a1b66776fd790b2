"""The Node host side on the CPU: the N-API addon (g4hip.node) and
HipBackend (gemma4-webgpu_amd/node/hip_backend.js), checked by
tests/node/test_napi_cpu.js under Node; and the addon's GGUF keys with the
backend's configFromGGUF against the Python reader on the same files
(tests/node/gguf_read.js)."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from g4hip.gguf import GGUFFile, config_from_gguf
from gguf_writer import ARR, BOOL, F32, GGUFWriter, I32, I64, STR, U32, U64

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "gemma4-webgpu_amd", "node", "g4hip.node")


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
def test_node_addon_and_backend_on_cpu():
    assert os.path.exists(ADDON), "g4hip.node is not built (run __graft_entry__.build())"
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "test_napi_cpu.js")], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all node CPU checks passed" in r.stdout


def _e2b_file(path: str) -> str:
    n = 6
    w = GGUFWriter(alignment=64)
    w.kv("general.architecture", STR, "gemma4")
    w.kv("gemma4.embedding_length", U32, 1536).kv("gemma4.block_count", U32, n)
    w.kv("gemma4.attention.head_count", U32, 8).kv("gemma4.attention.head_count_kv", U32, 1)
    w.kv("gemma4.context_length", U32, 131072)
    w.array("gemma4.feed_forward_length", I32, [6144] * 3 + [12288] * 3)
    w.kv("gemma4.attention.key_length", U32, 512).kv("gemma4.attention.key_length_swa", U32, 256)
    w.kv("gemma4.rope.freq_base", F32, 1e6).kv("gemma4.rope.freq_base_swa", F32, 1e4)
    w.kv("gemma4.attention.sliding_window", U32, 512)
    w.array("gemma4.attention.sliding_window_pattern", BOOL, [True, False, True, True, False, True])
    w.kv("gemma4.embedding_length_per_layer_input", U32, 256)
    w.kv("gemma4.final_logit_softcapping", F32, 30.0)
    w.kv("gemma4.attention.shared_kv_layers", U32, 3)
    w.kv("big.u64", U64, 2**63 + 11).kv("big.i64", I64, -(2**62) - 3)
    w.array("tokenizer.ggml.tokens", STR, ["<pad>", "é", "x" * 300])
    rng = np.random.default_rng(3)
    w.tensor("token_embd.weight", (256, 2), 14, rng.integers(0, 256, 2 * 210, dtype=np.uint8))
    w.tensor("output_norm.weight", (5,), 0, rng.standard_normal(5).astype(np.float32))
    w.tensor("blk.0.attn_q.weight", (512, 3), 12, rng.integers(0, 256, 6 * 144, dtype=np.uint8))
    return w.write(path)


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
def test_node_gguf_keys_match_the_python_reader(tmp_path):
    assert os.path.exists(ADDON), "g4hip.node is not built (run __graft_entry__.build())"
    path = _e2b_file(str(tmp_path / "m.gguf"))
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "gguf_read.js"), path, "8192"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    js = json.loads(r.stdout)
    g = GGUFFile(path)
    assert js["info"] == {"version": g.version, "tensorCount": g.tensor_count, "kvCount": g.kv_count,
                          "dataOffset": g.data_offset, "alignment": g.alignment}
    names = {0: "uint8", 1: "int8", 2: "uint16", 3: "int16", 4: "uint32", 5: "int32", 6: "float32", 7: "bool",
             8: "string", 9: "array", 10: "uint64", 11: "int64", 12: "float64"}
    for k, (t, v) in g.kv.items():
        e = js["meta"][k]
        assert e["type"] == names[t], k
        if t == ARR:
            assert [x["value"] for x in e["value"]] == v, k
        elif t in (10, 11):
            assert int(e["value"]) == v, k
        elif t == F32:
            assert np.float32(e["value"]) == np.float32(v), k
        else:
            assert e["value"] == v, k
    assert [(t["name"], t["dims"], t["type"], t["offset"], t["nbytes"]) for t in js["tensors"]] == \
        [(t.name, list(t.dims), t.type, t.offset, t.nbytes) for t in g.tensors]
    cfg = config_from_gguf(g, 8192)
    c = js["config"]
    pairs = {"hidden_size": "hidden_size", "num_layers": "num_layers", "num_q_heads": "num_q_heads",
             "num_kv_heads": "num_kv_heads", "context_length": "context_length",
             "intermediate_sizes": "intermediate_sizes", "head_dim_global": "head_dim_global",
             "head_dim_local": "head_dim_local", "rope_theta_global": "rope_theta_global",
             "rope_theta_swa": "rope_theta_swa", "sliding_window": "sliding_window",
             "attention_is_sliding": "attention_is_sliding", "per_layer_input_dim": "per_layer_input_dim",
             "final_logit_softcapping": "final_logit_softcapping", "num_unshared_layers": "num_unshared_layers",
             "kv_producer_for_layer": "kv_producer_for_layer"}
    for jk, pk in pairs.items():
        assert c[jk] == cfg[pk], jk
    assert js["openError"] == "G4_ERR_INVALID"
