"""Writes the committed golden fixtures of the attention path from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its only known-answer
test, test_olmo_model.cpp:48-70, needs trained weights that are Git-LFS
pointers in the reference checkout), so these fixtures are oracle outputs on
the seeded workloads. The oracle itself is pinned independently in
tests/test_oracle_pins.py; the fixtures anchor it against regressions and give
the GPU tests known answers.

Fixtures:
  flash_config1_fp32.npz  O, m, l for B=1, T=64, H=16, D=128, causal, seeds 1001-1003
  norm_rope_small.npz     q/k projections [1, 8, 2048] (seeds 601/602), norm weights of the
                          layer workload, and the fused RMSNorm + RoPE outputs and rms
  layer_small.npz         OlmoAttention forward of x [1, 16, 2048] (seed 2001) with the layer
                          workload's weights (seeds 2011-2014, 2021-2022)
  rope_table_checks.npz   selected rows of the fp64-derived sin/cos tables (theta 5e5)
  synth_checks.npz        first values of the seeded generators
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from dirktensor_amd import synth  # noqa: E402

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))
ROPE_ROWS = np.array([0, 1, 2, 63, 511, 4095, 6143, 8191])


def main():
    Q, K, V = synth.qkv(1, 64, 16)
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE, nthreads=1)
    np.savez_compressed(os.path.join(HERE, "flash_config1_fp32.npz"), O=O, m=m, l=l)

    w = synth.attention_layer_weights()
    q = synth.normal(601, (1, 8, 2048))
    k = synth.normal(602, (1, 8, 2048))
    s, c = oracle.rope_tables(8)
    qn, q_rms = oracle.rmsnorm_forward(q, w["q_norm"])
    kn, k_rms = oracle.rmsnorm_forward(k, w["k_norm"])
    qr = oracle.apply_rope(qn.reshape(1, 8, 16, 128), s, c)
    kr = oracle.apply_rope(kn.reshape(1, 8, 16, 128), s, c)
    np.savez_compressed(os.path.join(HERE, "norm_rope_small.npz"), q_out=qr, k_out=kr, q_rms=q_rms, k_rms=k_rms)

    x = synth.layer_input(1, 16)
    out = oracle.attention_layer_forward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"],
                                         nthreads=1)
    np.savez_compressed(os.path.join(HERE, "layer_small.npz"), out=out)

    s, c = oracle.rope_tables(8192)
    np.savez_compressed(os.path.join(HERE, "rope_table_checks.npz"), rows=ROPE_ROWS, sin=s[ROPE_ROWS],
                        cos=c[ROPE_ROWS])

    np.savez_compressed(os.path.join(HERE, "synth_checks.npz"), splitmix_seed1001=synth.splitmix64(1001, 8),
                        normal_seed1001=synth.normal(1001, (16,)), lengths_seed4001=synth.ragged_lengths())
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
