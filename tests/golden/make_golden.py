"""Writes the committed golden fixtures from the float64 oracle.

    python tests/golden/make_golden.py

cpu_plumbing_B1_H4_S256_D64.npz
    The CPU plumbing workload: Q, K, V ~ N(0,1) float32 from numpy default_rng(0),
    drawn in the order Q, K, V, shape [1, 4, 256, 64] (stored as the SHA-256 of their
    bytes; the arrays are regenerated from the seed); O = causal attention in float64
    (stored as float32) and LSE in the base-2 units of the backward's forward.
tiny_grads_B1_H2_S16_D8.npz
    A tiny case with dO and the float64 gradients, for the backward's known answers.
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention_oracle as orc  # noqa: E402
from oracle import cases  # noqa: E402


def main():
    q, k, v = cases.normal_inputs([(1, 4, 256, 64)] * 3, seed=0)
    o = orc.forward(q, k, v)
    digest = np.frombuffer(hashlib.sha256(q.tobytes() + k.tobytes() + v.tobytes()).digest(), np.uint8)
    np.savez_compressed(os.path.join(HERE, "cpu_plumbing_B1_H4_S256_D64.npz"), QKV_SHA256=digest,
                        O=o.astype(np.float32), LSE=orc.lse_log2(q, k).astype(np.float32))
    q, k, v, do = cases.normal_inputs([(1, 2, 16, 8)] * 4, seed=7)
    o, dq, dk, dv = orc.backward(q, k, v, do)
    np.savez_compressed(os.path.join(HERE, "tiny_grads_B1_H2_S16_D8.npz"), Q=q, K=k, V=v, dO=do,
                        O=o, dQ=dq, dK=dk, dV=dv, LSE=orc.lse_log2(q, k))


if __name__ == "__main__":
    main()
