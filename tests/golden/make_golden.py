"""Extracts the data arrays the tests pin against from the reference's own
fixture files (public/ref/layer_0_detail.npz and public/ref/smoke.npz, HF bf16
activations of Gemma-4-E2B at position 14 of the canonical prompt) into
tests/golden/ref_fixtures.npz.

Only data is copied (numpy arrays loaded with allow_pickle=False); no
reference code is run. Re-run with the reference checked out at
/root/reference:  python tests/golden/make_golden.py
"""
import hashlib
import os

import numpy as np

REF = os.environ.get("G4_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))

LAYER0 = [
    "L0_self_attn.v_proj_output",
    "L0_self_attn.v_norm_output",
    "L0_self_attn.q_proj_output",
    "L0_self_attn.q_norm_output",
    "L0_self_attn.k_proj_output",
    "L0_self_attn.k_norm_output",
    "L0_mlp.gate_proj_output",
    "L0_mlp.act_fn_output",
    "L0_mlp.up_proj_output",
    "L0_mlp_down_proj_input",
]
SMOKE = ["tokens", "position", "logits_pos14"]


def main():
    l0 = np.load(os.path.join(REF, "public/ref/layer_0_detail.npz"), allow_pickle=False)
    sm = np.load(os.path.join(REF, "public/ref/smoke.npz"), allow_pickle=False)
    out = {}
    for k in LAYER0:
        out[k.replace(".", "__")] = l0[k]
    for k in SMOKE:
        out[k] = sm[k]
    path = os.path.join(HERE, "ref_fixtures.npz")
    np.savez_compressed(path, **out)
    h = hashlib.sha256(open(path, "rb").read()).hexdigest()
    print(f"wrote {path} ({os.path.getsize(path)} bytes) sha256={h}")


if __name__ == "__main__":
    main()
