"""Write the committed golden vectors (run from the repo root):

    python tests/golden/make_golden.py

cfg0.npz        BASELINE config 0: B=1, T=256, H=4 (qk = v heads), K=V=64,
                zero initial state, seed 0.
varlen_h0.npz   B=1, T=150 packed as cu_seqlens [0, 40, 40, 101, 150],
                Hqk=2 -> Hv=4, K=V=64, initial state 0.01 N(0,1), seed 1.

Inputs come from avelang_amd.workloads (numpy PCG64); q, k, v are stored
as bf16 bit patterns (uint16), g / beta / h0 as fp32.  Expected o and final
state come from the fp64 per-token recurrence of oracle/gdn_ref.py (the
definition), stored as fp32.  ``sha256.json`` holds the input digests.
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from avelang_amd import workloads as W  # noqa: E402
from oracle import gdn_ref  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def bits(x):
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def write(name, wl):
    a = wl.numpy()
    o, s = gdn_ref.recurrent(**a, dtype=np.float64)
    arrs = dict(q_bf16=bits(a["q"]), k_bf16=bits(a["k"]), v_bf16=bits(a["v"]),
                g=a["g"], beta=a["beta"], o=o.astype(np.float32), state=s.astype(np.float32))
    if a["initial_state"] is not None:
        arrs["h0"] = a["initial_state"]
    if a["cu_seqlens"] is not None:
        arrs["cu_seqlens"] = a["cu_seqlens"]
    np.savez_compressed(os.path.join(HERE, name), **arrs)
    h = hashlib.sha256()
    for key in sorted(k for k in arrs if k not in ("o", "state")):
        h.update(np.ascontiguousarray(arrs[key]).tobytes())
    return h.hexdigest()


def main():
    digests = {
        "cfg0.npz": write("cfg0.npz", W.config("cfg0_cpu_reference", seed=0)),
        "varlen_h0.npz": write("varlen_h0.npz", W.make(
            1, 150, 2, 4, 64, 64, seed=1, h0_scale=0.01,
            cu_seqlens=np.array([0, 40, 40, 101, 150], np.int32))),
    }
    with open(os.path.join(HERE, "sha256.json"), "w") as f:
        json.dump(digests, f, indent=1, sort_keys=True)
    print(digests)


if __name__ == "__main__":
    main()
