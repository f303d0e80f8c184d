"""Writes tests/golden/zipf_routing.npz: for each Zipf-skewed benchmark
configuration (c3, c5) the per-expert router logit bias that gives its
top-K load a Zipf(alpha) shape over a seeded permutation of the experts,
and the per-expert row counts the block's routing realises at each of the
configuration's token counts (x seeded with T, as the bench and the
parity tests draw it).

The bias is calibrated once, here, by fixed-point iterations
b += (log p - log p_hat) / 2 on a calibration batch of 4096 tokens (seed 1)
through the router's f32 logits; workloads.make_weights then loads it, so
the c3/c5 routing no longer depends on the calibration's own arithmetic.
The row counts pin the whole routing chain: the GPU parity tests compare
the block's realised load with them.  Needs a GPU (the weights are drawn by
torch's device generator):

    python tests/golden/make_zipf_routing.py [--out DIR]
"""
from __future__ import annotations

import argparse
import shutil
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
FIXTURE = Path(__file__).resolve().parent / "zipf_routing.npz"


def calibrate(W, cfg, gate_w, device, iters=20, n_cal=4096):
    E, K = cfg.E, cfg.K
    perm = torch.randperm(E, generator=W._gen("cpu", cfg.seed, 7))
    rank = torch.empty(E)
    rank[perm] = torch.arange(1, E + 1, dtype=torch.float32)
    p = rank.pow(-cfg.zipf_alpha)
    p = (p / p.sum()).to(device)
    b = p.log()
    xc = W._normal((n_cal, cfg.d), 1.0, device, 1, 11).to(torch.bfloat16).float()
    base = xc @ gate_w.t()
    for _ in range(iters):
        top = (base + b).topk(K, dim=-1).indices
        load = torch.bincount(top.reshape(-1), minlength=E).float() / (n_cal * K)
        if (load - p).abs().sum() < 0.05:
            break
        b = b + (p.log() - (load + 1e-6).log()) * 0.5
    return b.float().cpu().numpy(), perm.numpy().astype(np.int32)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--out", default=None, help="also copy the fixture into this directory")
    ap.add_argument("--rows-only", action="store_true",
                    help="keep the committed bias and permutation; record only the row "
                         "counts the current routing realises")
    args = ap.parse_args()
    import __graft_entry__ as entry
    pkg = entry.load_package()
    W = pkg.workloads
    dev = torch.device("cuda:0")
    keys = [k for k, c in W.CONFIGS.items() if c.zipf_alpha]
    data = {}
    if args.rows_only:
        with np.load(FIXTURE) as z:
            data = {f: z[f] for f in z.files if f.endswith("__bias") or f.endswith("__perm")}
    else:
        for k in keys:
            cfg = W.CONFIGS[k]
            gate_w = W._normal((cfg.E, cfg.d), 0.02, dev, cfg.seed, 2)
            bias, perm = calibrate(W, cfg, gate_w, dev)
            data[f"{cfg.name}__bias"] = bias
            data[f"{cfg.name}__perm"] = perm
            print(f"{k}: bias [{bias.min():.3f}, {bias.max():.3f}]", flush=True)
        np.savez(FIXTURE, **data)
    # the realised load of each token count, through the block's routing
    for k in keys:
        cfg = W.CONFIGS[k]
        bw = W.make_weights(cfg, dev)
        block = bw.block()
        for T in cfg.tokens:
            block(W.make_x(cfg, T, dev, seed=T))
            h = torch.bincount(block.last_indices.reshape(-1).long(), minlength=cfg.E)
            data[f"{cfg.name}__rows_T{T}"] = h.cpu().numpy().astype(np.int32)
            print(f"{k} T={T}: rows max {int(h.max())} min {int(h.min())}", flush=True)
        del bw, block
        torch.cuda.empty_cache()
    np.savez(FIXTURE, **data)
    if args.out:
        Path(args.out).mkdir(parents=True, exist_ok=True)
        shutil.copy(FIXTURE, Path(args.out) / FIXTURE.name)
    print(f"wrote {FIXTURE}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
