"""A minimal safetensors writer for the checkpoint tests (the format: an
8-byte little-endian header length, the JSON header, then the tensors'
bytes), and a model directory of shards plus model.safetensors.index.json
in the Hugging Face layout."""
import json
import os
import struct

import numpy as np


def write_safetensors(path, tensors, pad=8):
    """tensors: {name: (dtype "BF16"/"F16"/"F32", numpy array)}; arrays of
    bf16 are uint16 bits."""
    header, blobs, at = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dt, a) in tensors.items():
        raw = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [at, at + len(raw)]}
        blobs.append(raw)
        at += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % pad)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def write_model(dirpath, shards):
    """shards: [{name: (dtype, array)}, ...] as model-0000i-of-0000n.safetensors
    with the index mapping every name to its shard."""
    os.makedirs(dirpath, exist_ok=True)
    wm = {}
    for i, t in enumerate(shards):
        fn = "model-%05d-of-%05d.safetensors" % (i + 1, len(shards))
        write_safetensors(os.path.join(dirpath, fn), t)
        for name in t:
            wm[name] = fn
    with open(os.path.join(dirpath, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": wm}, f)
