"""Regenerate the committed golden vectors from the float64 oracle.

The reference ships no tests or fixtures, so these vectors come from this build's oracle
(oracle/nerf64.py), itself pinned by independent checks (tests/test_oracle.py).  They let
the GPU box compare against fixed numbers without running the oracle at large sizes.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import nerf64 as o  # noqa: E402

BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)


def make_c0() -> dict:
    # Config 0: B=1, N=64, float64, default anchors, seed 0.
    d = o.synthetic_inputs(1, 64, seed=0, anchors=False)
    xyz = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"])
    gL, gA, gD = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    return dict(lengths=d["lengths"], angles=d["angles"], dihedrals=d["dihedrals"], grad=d["grad"], xyz=xyz,
                grad_lengths=gL, grad_angles=gA, grad_dihedrals=gD)


def make_anchored() -> dict:
    # B=3, N=33 with explicit random anchors (config 2 anchor draw), seed 2.
    d = o.synthetic_inputs(3, 33, seed=2, anchors=True)
    an = dict(p0=d["p0"], first_direction=d["first_direction"], initial_normal=d["initial_normal"])
    xyz = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    gL, gA, gD = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **an)
    return dict(lengths=d["lengths"], angles=d["angles"], dihedrals=d["dihedrals"], grad=d["grad"], xyz=xyz,
                grad_lengths=gL, grad_angles=gA, grad_dihedrals=gD, **an)


def make_torsion() -> dict:
    # Config 3 constants, B=2, N=40, raw pairs ~N(0,1), seed 3.
    rng = np.random.default_rng(3)
    raw = rng.normal(size=(2, 2 * 37))
    grad = rng.normal(size=(2, 40, 3))
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    xyz = o.torsion_forward(raw, c)
    graw = o.torsion_backward(raw, xyz, grad, c)
    return dict(raw_pairs=raw, grad=grad, xyz=xyz, grad_raw=graw, bond_lengths=np.array(BOND_LENGTHS),
                bond_angles=np.array(BOND_ANGLES))


def main() -> None:
    np.savez(HERE / "c0_reconstruct.npz", **make_c0())
    np.savez(HERE / "anchored_reconstruct.npz", **make_anchored())
    np.savez(HERE / "torsion_small.npz", **make_torsion())


if __name__ == "__main__":
    main()
