"""Writes the committed golden fixtures of this directory from the oracle
(the C++ restatement of kestrel's CPU path: oracle/kmoe_oracle.cpp).

The reference ships no golden vectors for this path (its tests generate data
at run time and *.gguf files are ignored), and its Rust code cannot be built
here, so the fixtures pin the oracle's outputs on seeded inputs:

  manifest.json        seeds, generator, SHA-256 of every generated tensor and
                       of every output array
  c1_q8_0_moe.npz      config 1 (Q8_0, hidden 1024, FFN 512, 8 experts, top-2,
                       16 tokens): routing indices and weights, dispatch
                       permutation and offsets, fp32 output of the AVX2 regime
  c2_q4k_rows.npz      Q4_K rows of a 4096-wide matrix against one Q8_K row:
                       the activation quantization, per-superblock integer
                       accumulators (sumi, mins) and the int-path matvec

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

C1 = dict(n_expert=8, k=2, d=1024, ff=512, seed=0, tokens=16, h_seed=0)
C2 = dict(rows=8, cols=4096, w_seed=21, x_seed=22)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_inputs():
    from oracle import pyoracle as orc
    from tests.helpers import Q8_0, LayerSpec

    spec = LayerSpec(C1["n_expert"], C1["k"], C1["d"], C1["ff"], Q8_0, seed=C1["seed"])
    h = orc.normal(C1["h_seed"], C1["tokens"] * C1["d"]).reshape(C1["tokens"], C1["d"])
    return spec, h


def c2_inputs():
    from oracle import pyoracle as orc
    from tests.helpers import Q4_K, random_blocks

    w = random_blocks(Q4_K, C2["rows"], C2["cols"], C2["w_seed"])
    x = orc.normal(C2["x_seed"], C2["cols"]).reshape(1, C2["cols"])
    return w, x


def c1_outputs(spec, h):
    from oracle import pyoracle as orc

    L = spec.oracle_layer()
    idx, w = L.route(h, orc.REGIME_AVX2)
    perm, off = orc.dispatch(idx, spec.n_expert)
    out = L.moe_ffn(h, orc.REGIME_AVX2)
    return dict(idx=idx.astype(np.uint32), w=w.astype(np.float32), perm=perm.astype(np.uint32),
                offsets=off.astype(np.uint32), out=out.astype(np.float32))


def c2_outputs(w, x):
    from oracle import pyoracle as orc
    from tests.helpers import Q4_K, row_bytes

    q, d, bsums = orc.q8k_quantize(x)
    rb = row_bytes(Q4_K, C2["cols"])
    sumi, mins = [], []
    for r in range(C2["rows"]):
        s, m = orc.q4k_block_acc(w[r * rb:(r + 1) * rb], C2["cols"], q[0], bsums[0])
        sumi.append(s)
        mins.append(m)
    y = orc.matmul(Q4_K, w, C2["rows"], C2["cols"], x, orc.REGIME_INT8)
    return dict(xq=q.astype(np.int8), xd=d.astype(np.float32), bsums=bsums.astype(np.int32),
                sumi=np.asarray(sumi, np.int32), mins=np.asarray(mins, np.int32), y=y.astype(np.float32))


def input_hashes(spec, h, w2, x2) -> dict:
    return {
        "c1.router": sha(spec.router),
        "c1.gate": [sha(g) for g in spec.gate],
        "c1.up": [sha(u) for u in spec.up],
        "c1.down": [sha(d) for d in spec.down],
        "c1.h": sha(h),
        "c2.w": sha(w2),
        "c2.x": sha(x2),
    }


def main():
    spec, h = c1_inputs()
    w2, x2 = c2_inputs()
    o1 = c1_outputs(spec, h)
    o2 = c2_outputs(w2, x2)
    np.savez(os.path.join(HERE, "c1_q8_0_moe.npz"), **o1)
    np.savez(os.path.join(HERE, "c2_q4k_rows.npz"), **o2)
    manifest = {
        "generator": "splitmix64 -> uniform (0,1) -> Box-Muller in double (oracle orc_fill_normal); "
                     "weights: the oracle's Q8_0 quantizer on N(0, 0.02) (config 1), random well-formed "
                     "Q4_K blocks with d = 1.4e-4, dmin = 7.5 d (config 2 rows)",
        "c1": C1,
        "c2": C2,
        "inputs_sha256": input_hashes(spec, h, w2, x2),
        "outputs_sha256": {**{f"c1.{k}": sha(v) for k, v in o1.items()}, **{f"c2.{k}": sha(v) for k, v in o2.items()}},
    }
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
