"""Writes tests/golden/c1_block.npz: the c1 block (T=16, d=512, E=8, K=2,
f=256, 4-bit g64, seed 0) run through the CPU oracle.

Inputs are regenerated from numpy's PCG64 stream (seed 0) by
`c1_inputs()`, so the fixture stores only their SHA-256 digests and the
expected routing and output.  Run from the repository root:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as orc  # noqa: E402

OUT = Path(__file__).resolve().parent / "c1_block.npz"
D, E, K, F, T = 512, 8, 2, 256, 16


def c1_inputs(seed: int = 0):
    """x bf16 [T, d]; router f32 [E, d]; gate/up/down quantised (4-bit g64)."""
    rng = np.random.default_rng(seed)
    x = orc.f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32))
    router = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)

    def bank(shape):
        w = orc.f32_to_bf16((rng.standard_normal(shape) * 0.02).astype(np.float32))
        return w, orc.quantize(w, 64, 4)

    gate_w, gate = bank((E, F, D))
    up_w, up = bank((E, F, D))
    down_w, down = bank((E, D, F))
    params = dict(d=D, E=E, K=K, f=F, fs=0, bits=4, group_size=64, router_w=router,
                  router_b=None, gate=gate, up=up, down=down)
    dense = dict(gate=gate_w, up=up_w, down=down_w)
    return x, params, dense


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main():
    x, p, dense = c1_inputs()
    out, idx, w = orc.block_forward(p, x)
    np.savez(OUT, out=out, idx=idx, weights=w,
             x_sha=digest(x), router_sha=digest(p["router_w"]),
             dense_sha=digest(dense["gate"], dense["up"], dense["down"]),
             packed_sha=digest(*p["gate"], *p["up"], *p["down"]))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
