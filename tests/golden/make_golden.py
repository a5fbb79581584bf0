"""Write tests/golden/golden.npz: seeded inputs and the reference CPU route's
outputs for the small cases of oracle/ref_cases.py.

Expected outputs come from the reference's own ``cpu_einsum.h`` compiled by
oracle/ref_build.py (the reference ships no golden vectors of its own:
every reference test draws fresh ``torch.rand`` inputs).  float16 cases
store float16 inputs and the reference output on their float32 up-cast,
which is how parity is defined for float16 (the CPU route rejects float16,
builder.py:612-613).

Run from the repository root after ``python oracle/ref_build.py``:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import ref_build  # noqa: E402
from ref_cases import REF_CASES  # noqa: E402

MAX_ELEMS = 16000  # inputs + output per case, keeps the fixture file small
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def main():
    arrays = {}
    index = []
    rng = np.random.default_rng(20261201)
    for n, (eq, s0, s1) in enumerate(REF_CASES):
        r, _ = ref_build.oracle.cpu_plan(eq, s0, s1)
        total = int(np.prod(s0)) + int(np.prod(s1)) + int(np.prod(r["out_shape"]))
        if total > MAX_ELEMS:
            continue
        for dt in ("f32", "f16"):
            if dt == "f32":
                a = rng.standard_normal(s0).astype(np.float32)
                b = rng.standard_normal(s1).astype(np.float32)
                a32, b32 = a, b
            else:
                a = rng.standard_normal(s0).astype(np.float16)
                b = rng.standard_normal(s1).astype(np.float16)
                a32, b32 = a.astype(np.float32), b.astype(np.float32)
            out = ref_build.run(eq, a32, b32)
            key = f"c{len(index)}"
            arrays[key + "_a"] = a
            arrays[key + "_b"] = b
            arrays[key + "_out"] = out
            index.append(f"{key}|{eq}|{dt}")
    arrays["index"] = np.array(index)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {len(index)} golden cases to {OUT} ({os.path.getsize(OUT) / 1e6:.2f} MB)")


if __name__ == "__main__":
    main()
