"""Load a golden fixture: bf16 tensors are stored as uint16 bit patterns
(keys ending in ``_bf16``) and come back as torch.bfloat16 under the bare name."""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load(name):
    z = np.load(os.path.join(HERE, f"{name}.npz"))          # allow_pickle stays False
    out = {}
    for k in z.files:
        a = z[k]
        if k.endswith("_bf16"):
            out[k[:-5]] = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        elif a.ndim == 0:
            out[k] = a.item()
        else:
            out[k] = torch.from_numpy(a.copy())
    return out
