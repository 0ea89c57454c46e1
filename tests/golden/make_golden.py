"""Write the golden fixtures in tests/golden/*.npz.

Each fixture holds, for one seeded case from oracle/inputs.py: the SHA-256
digest of every input tensor (so a test can rebuild the inputs from the
recipe and prove they are the same bytes), the case recipe, and the expected
outputs: the appended pool rows and the fp32 attention output.  The
expected outputs come from the vectorised oracle after it has been checked
here against the scalar brute-force loops; nothing is written on a mismatch.

The reference repository has no kernel-level fixtures of its own (it has no
tests); these pin the oracle and the GPU path to one fixed set of numbers.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import inputs, paged_attention as ref  # noqa: E402

# name -> (kind, recipe kwargs for inputs.make_case or a config function)
CASES = {
    "config1_decode": ("decode", {"config": "config1", "seed": 0}),
    "decode_edges": ("decode", {"prior_lens": [0, 1, 14, 15, 16, 31, 47, 100], "seed": 5}),
    "mixed_small": ("mixed", {"prior_lens": [0, 5, 20, 37, 0], "new_lens": [17, 1, 3, 1, 0], "seed": 3}),
}


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def build_case(spec: dict) -> inputs.PagedCase:
    spec = dict(spec)
    if "config" in spec:
        return getattr(inputs, spec.pop("config"))(**spec)
    return inputs.make_case(spec.pop("prior_lens"), spec.pop("new_lens", None), **spec)


INPUT_FIELDS = ("q", "k_new", "v_new", "k_pool", "v_pool", "block_table", "lens_pool",
                "slot_ids", "kv_lens", "new_lens", "cu_seqlens", "pages", "offsets")


def expected(kind: str, case: inputs.PagedCase) -> dict:
    kp, vp = case.appended_pools()
    out = {
        "k_rows": kp[case.pages, :, case.offsets].float().numpy(),
        "v_rows": vp[case.pages, :, case.offsets].float().numpy(),
        "pool_digest_k": digest(kp),
        "pool_digest_v": digest(vp),
    }
    if kind == "decode":
        o = ref.decode_attention(case.q, kp, vp, case.attended, case.slot_ids, case.block_table)
        brute = ref.decode_attention_bruteforce(case.q, kp, vp, case.attended, case.slot_ids,
                                                case.block_table)
        assert (o - brute).abs().max() < 1e-5, "oracle disagrees with brute force"
    else:
        o, written = ref.mixed_attention(case.q, kp, vp, case.cu_seqlens, case.kv_lens,
                                         case.slot_ids, case.block_table)
        brute = ref.mixed_attention_bruteforce(case.q, kp, vp, case.cu_seqlens, case.kv_lens,
                                               case.slot_ids, case.block_table)
        assert (o - brute)[written].abs().max() < 1e-5, "oracle disagrees with brute force"
        out["written"] = written.numpy()
    out["out"] = o.numpy()
    return out


def main() -> None:
    for name, (kind, spec) in CASES.items():
        case = build_case(spec)
        exp = expected(kind, case)
        arrays = {k: v for k, v in exp.items() if isinstance(v, np.ndarray)}
        meta = {
            "kind": kind,
            "spec": spec,
            "digests": {f: digest(getattr(case, f)) for f in INPUT_FIELDS},
            "pool_digest_k": exp["pool_digest_k"],
            "pool_digest_v": exp["pool_digest_v"],
        }
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, meta=np.array(json.dumps(meta)), **arrays)
        print(f"wrote {path}")


if __name__ == "__main__":
    main()
