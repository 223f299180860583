"""Writes the golden vectors under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

Inputs come from the package's seeded CPU generators (flash_gmm.data) and are
identified in each fixture by the SHA-256 of their float32 bytes, so a change
in torch's CPU generator is detected instead of silently changing the case.
Expected outputs are the float64 oracle (oracle/gmm_oracle.py), whose own
correctness is pinned by tests/test_oracle.py (scipy, sklearn, brute force).
"""

import hashlib
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "flash-gmm_amd"), ROOT]

from flash_gmm import data  # noqa: E402
from oracle import gmm_oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

CASES = {
    # name: (generator, sizes, seed, kind)
    "iso_n10k_k64_d32": (data.iso_plain, dict(N=10_000, K=64, D=32), 0, "iso"),
    "iso_clustered_n4096_k96_d40": (data.iso_clustered, dict(N=4096, K=96, D=40), 1, "iso"),
    "diag_n3000_k40_d24": (data.diag_clustered, dict(N=3000, K=40, D=24), 2, "diag"),
    "full_n2000_k12_d16": (data.full_clustered, dict(N=2000, K=12, D=16), 3, "full"),
}


def input_digest(inp):
    h = hashlib.sha256()
    for k in sorted(inp):
        h.update(k.encode())
        h.update(inp[k].detach().cpu().float().contiguous().numpy().tobytes())
    return h.hexdigest()


def make_inputs(name):
    fn, sizes, seed, kind = CASES[name]
    return fn(seed=seed, device="cpu", **sizes), kind


def expected(inp, kind):
    if kind == "iso":
        return O.estep_iso(inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
    if kind == "diag":
        return O.estep_diag(inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
    return O.estep_full(inp["X"], inp["mu"], inp["prec_chol"], inp["log_pi"])


def main():
    for name in CASES:
        inp, kind = make_inputs(name)
        logZ, Nk, mu_acc, sig = expected(inp, kind)
        path = os.path.join(OUT, name + ".npz")
        np.savez_compressed(path, sha256=np.array(input_digest(inp)), kind=np.array(kind),
                            logZ=logZ.numpy(), Nk=Nk.numpy(), mu_acc=mu_acc.numpy(), sig=sig.numpy())
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
