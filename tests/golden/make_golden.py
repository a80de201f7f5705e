"""Writes tests/golden/attn_hashes.json: blake2b-32 digests of the seeded
inputs and of the CPU oracle's outputs for a few fixed cases.

    python tests/golden/make_golden.py          # rewrite the fixture
    python tests/golden/make_golden.py --check  # compare, exit 1 on a difference

The reference holds no golden vectors for attention; these digests pin this
project's contract against regressions (a change of the contract changes
them, deliberately).  Digest framing follows the reference's state hash
(src/pretrain/train/state_hash.py:106-113): tag, dtype string, NUL, shape
string, NUL, raw little-endian bytes; blake2b with a 32-byte digest.
"""

from __future__ import annotations

import hashlib
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
FIXTURE = HERE / "attn_hashes.json"

# name: (B, H, Hkv, S, D, window, dtype, seed, rope_theta, qk_scale, backward)
CASES = {
    "c1_fwd_fp32": (1, 4, 4, 256, 64, 0, "f32", 1, None, None, False),
    "bf16_rope_fwd_bwd": (1, 2, 2, 128, 128, 0, "bf16", 2, 10000.0, None, True),
    "bf16_gqa_window_fwd_bwd": (2, 4, 2, 192, 64, 64, "bf16", 3, None, None, True),
    "bf16_qk_x3_fwd_bwd": (1, 2, 2, 256, 128, 0, "bf16", 4, None, 3.0, True),
}


def digest(tag: str, a: np.ndarray, dtype: str) -> str:
    """blake2b-32 of one tensor; ``dtype`` 'bf16' hashes the bf16 bytes."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == "bf16":
        raw = (a.view(np.uint32) >> 16).astype("<u2").tobytes()
        dname = "torch.bfloat16"
    else:
        raw = a.astype("<f4").tobytes()
        dname = "torch.float32"
    h = hashlib.blake2b(digest_size=32)
    h.update(tag.encode())
    h.update(dname.encode())
    h.update(b"\0")
    h.update(str(tuple(a.shape)).encode())
    h.update(b"\0")
    h.update(raw)
    return h.hexdigest()


def case_inputs(name: str) -> dict:
    """Seeded inputs of one case (binary32 arrays holding ``dtype`` values)."""
    sys.path.insert(0, str(ROOT))
    import __graft_entry__

    __graft_entry__.load_package()
    from open_transformers_amd import synthetic

    B, H, Hkv, S, D, w, dt, seed, theta, qks, bwd = CASES[name]
    return synthetic.make_inputs(B, H, Hkv, S, D, dtype=dt, seed=seed, rope_theta=theta, qk_scale=qks)


def digests(name: str, inp: dict, outs: dict) -> dict:
    """Digests of one case's inputs and of the outputs present in ``outs``."""
    dt = CASES[name][6]
    rec = {n: digest(n, inp[n], dt) for n in ("q", "k", "v", "do")}
    for n, a in outs.items():
        rec[n] = digest(n, a, "f32" if n == "lse" else dt)
    return rec


def compute_case(name: str) -> dict:
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc

    w, dt, bwd = CASES[name][5], CASES[name][6], CASES[name][10]
    inp = case_inputs(name)
    bf = dt == "bf16"
    o, lse = orc.attn_fwd(inp["q"], inp["k"], inp["v"], window=w, out_bf16=bf)
    outs = {"o": o, "lse": lse}
    if bwd:
        dq, dk, dv = orc.attn_bwd(inp["q"], inp["k"], inp["v"], o, lse, inp["do"], window=w, out_bf16=bf)
        outs.update(dq=dq, dk=dk, dv=dv)
    return digests(name, inp, outs)


def compute() -> dict:
    return {name: compute_case(name) for name in CASES}


def main() -> int:
    got = compute()
    if "--check" in sys.argv:
        want = json.loads(FIXTURE.read_text())
        bad = [(c, t) for c in want for t in want[c] if got.get(c, {}).get(t) != want[c][t]]
        for c, t in bad:
            print(f"differs: {c}/{t}")
        return 1 if bad else 0
    FIXTURE.write_text(json.dumps(got, indent=1, sort_keys=True) + "\n")
    print(f"wrote {FIXTURE}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
