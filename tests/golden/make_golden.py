"""Writes tests/golden/mlp784-128-128-10_b64_sgd.npz: the oracle's result for one step of
the 784-128-128-10 MLP, batch 64, SGD(lr=0.1) on the seeded inputs of
orcaml_amd.synth (seed 1).  Inputs are not stored: the fixture records the
labels and the sum of x so the generator itself is pinned too.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from orcaml_amd import synth  # noqa: E402


def main() -> None:
    w = synth.WORKLOADS[synth.MLP_SMALL]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    r = O.mlp_train(w["dims"], params, x, onehot, O.make_opt("sgd", 0.1), steps=1)
    out = dict(labels=labels, x_sum=np.float64(x.astype(np.float64).sum()), loss=r["losses"], logits=r["logits"],
               preds=r["preds"], correct=np.int64(r["correct"]))
    for i in range(6):
        out[f"grad{i}"] = r["grads"][i]
        out[f"param{i}"] = r["params"][i]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mlp784-128-128-10_b64_sgd.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: loss {float(r['losses'][0]):.7f}, correct {r['correct']}")


if __name__ == "__main__":
    main()
