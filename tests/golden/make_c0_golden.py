"""Writes the config-0 golden vectors (tests/golden/c0/*.ds5t) from the CPU oracle.

Config 0 is the CPU-reference fixture decode step: Qwen3-30B-A3B attention shape
(32 q heads, 4 kv heads, head_dim 128), q/k/v f32 N(0,1) from seed 0, norm weights
N(1, 0.02), eps 1e-6, theta 1e6, f16 cache of capacity 32 holding 31 tokens; the
step appends token 31 and attends over 32. Inputs come from qw3_amd.synth; the
expected outputs (cache after the append, attention output) from the oracle's
engine-order step (oracle/ds5_oracle.c ds5o_attention_step).

    python tests/golden/make_c0_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from qw3_amd import synth  # noqa: E402

OUT = os.path.join(HERE, "c0")


def make():
    cfg = synth.CONFIGS[0]
    s, cap, pos = cfg["shape"], cfg["cap"], cfg["pos"]
    q, k, v, qn, kn = synth.step_inputs(0, 0, 1, s)
    kc, vc = synth.cache_f16(0, 0, s, cap, pos)
    positions = np.array([pos], np.int32)
    kc_out, vc_out = kc.copy(), vc.copy()
    out, q_rot, k_rot = O.attention_step(q, k, v, qn, kn, positions, kc_out, vc_out, kv_dtype=1, pos=pos,
                                         n_tokens=1, n_q_heads=s.n_q_heads, n_kv_heads=s.n_kv_heads,
                                         head_dim=s.head_dim, max_ctx=cap, eps=s.eps, theta=s.theta,
                                         scale=s.scale)
    return {
        "q": (q, O.F32), "k": (k, O.F32), "v": (v, O.F32), "q_norm": (qn, O.F32), "k_norm": (kn, O.F32),
        "positions": (positions, O.I32), "k_cache_in": (kc, O.F16), "v_cache_in": (vc, O.F16),
        "k_cache_out": (kc_out, O.F16), "v_cache_out": (vc_out, O.F16), "q_rot": (q_rot, O.F32),
        "k_rot": (k_rot, O.F32), "output": (out.reshape(1, -1), O.F32),
    }


if __name__ == "__main__":
    os.makedirs(OUT, exist_ok=True)
    for name, (arr, dt) in make().items():
        O.write_ds5t(os.path.join(OUT, f"{name}.ds5t"), arr, dt)
    print("wrote", OUT)
