"""Writes the small golden fixtures of tests/golden/ from the CPU oracle.

Each fixture is one short iPC trajectory: seeded inputs (weights, batch),
the forward-initialised states, and the states, errors and weights after T
steps, all fp32, stored with numpy.savez_compressed.  The oracle itself is
pinned by tests/test_oracle.py; these files freeze its output so that later
changes to the oracle or the HIP path are compared with fixed numbers.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import ipc_oracle as O  # noqa: E402

CASES = {
    # name: (dims, batch, activation, T, init, input distribution, seed)
    "c1_like_tanh": ((10, 32, 32, 48), 16, "tanh", 4, "xavier_uniform", "uniform", 0),
    "deep_relu": ((4, 16, 16, 16, 16, 24), 8, "relu", 5, "kaiming_a_sqrt5", "uniform", 1),
    "gelu_b1": ((3, 8, 8, 12), 1, "gelu", 6, "xavier_uniform", "normal", 2),
    "sigmoid_ragged": ((7, 13, 9, 21), 5, "sigmoid", 3, "kaiming_a_sqrt5", "normal", 3),
}


def make(name, dims, B, act, T, init, dist, seed):
    w0 = O.init_weights(dims, seed=seed, init=init)
    x_in, labels, y = O.make_batch(dims, B, seed=seed, input_dist=dist)
    x0 = O.forward_init(x_in, y, w0, act)
    xt, wt, et = O.run_steps(x0, w0, T, act=act, alpha=1e-3, gamma=0.5)
    out = {"dims": np.array(dims, dtype=np.int64), "batch": np.int64(B), "steps": np.int64(T),
           "alpha": np.float64(1e-3), "gamma": np.float64(0.5), "act": np.array(act),
           "x_in": x_in.numpy(), "y": y.numpy()}
    for l, w in enumerate(w0):
        out[f"w0_{l}"] = w.numpy()
        out[f"wT_{l}"] = wt[l].numpy()
        out[f"eT_{l}"] = et[l].numpy()
    for l, x in enumerate(x0):
        out[f"x0_{l}"] = x.numpy()
        out[f"xT_{l}"] = xt[l].numpy()
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)


if __name__ == "__main__":
    torch.set_num_threads(1)
    for name, spec in CASES.items():
        make(name, *spec)
        print("wrote", name)
