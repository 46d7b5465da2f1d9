"""Reader for tests/golden/attn_small.json (written by make_golden.py)."""
import base64
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _tensor(obj):
    if obj is None:
        return None
    if "q8" in obj:
        raw = np.frombuffer(base64.b64decode(obj["q8"]), dtype=np.int8)
        arr = raw.astype(np.float32) / 8.0
    else:
        arr = np.frombuffer(base64.b64decode(obj["f32"]), dtype="<f4")
    return torch.from_numpy(arr.copy()).reshape(obj["shape"])


def cases(kind=None):
    with open(os.path.join(HERE, "attn_small.json")) as f:
        data = json.load(f)
    out = []
    for c in data["cases"]:
        if kind and c["kind"] != kind:
            continue
        d = dict(c)
        for key in ("q", "k", "v", "k_pool", "v_pool", "rel", "pool", "want",
                    "out", "lse"):
            if isinstance(d.get(key), dict):
                d[key] = _tensor(d[key])
        for key in ("q", "k", "v", "k_pool", "v_pool", "rel"):
            if d.get(key) is not None:
                d[key] = d[key].to(torch.bfloat16)   # exact: multiples of 1/8
        out.append(d)
    return out
