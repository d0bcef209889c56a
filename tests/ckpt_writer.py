# SPDX-License-Identifier: Apache-2.0
"""A synthetic checkpoint in the packer's expert layout, for the loader tests.

Writes what tools/pack_trunk.py and the model's shards give the reference's
reader (src/40_io/dsv4_st.c:60-135): index_dir/experts.idx (b"DSV4EXP1",
int32 n_layers and n_experts, then n_layers x n_experts x 6 little-endian
records "<iiqq" = shard, pad, offset, bytes, tensors in the order w1, w1
scales, w2, w2 scales, w3, w3 scales; tools/pack_trunk.py:333-346) and shard
files named *.safetensors, read as raw bytes at the recorded offsets (the
reader never parses their headers), tensors scattered over the shards with
filler between them."""
import os
import struct

import numpy as np

import pyoracle as P


def write_checkpoint(orc, root, n_layers, n_experts, hidden, inter, seed, n_shards=3):
    """Returns {(layer, expert): HostExpert} of what was written."""
    rng = np.random.default_rng(seed)
    model_dir = os.path.join(root, "model")
    index_dir = os.path.join(root, "index")
    os.makedirs(model_dir, exist_ok=True)
    os.makedirs(index_dir, exist_ok=True)
    names = [f"model-{i + 1:05d}-of-{n_shards:05d}.safetensors" for i in range(n_shards)]
    # shard order is strcmp order of the paths; write them in another order
    shard_bytes = [bytearray(rng.integers(0, 256, 64, dtype=np.uint8).tobytes()) for _ in names]
    records, hosts = [], {}
    for L in range(n_layers):
        for E in range(n_experts):
            mats = []
            for (r, c) in ((inter, hidden), (hidden, inter), (inter, hidden)):    # w1, w2, w3
                w = (rng.standard_normal((r, c)) * 0.02).astype(np.float32)
                W, S = orc.quant_fp4_mx(w)
                mats.append((W, S, r, c))
            for (W, S, r, c) in mats:                   # index order: w, then its scales
                for arr in (W, S):
                    sh = int(rng.integers(0, n_shards))
                    pad = int(rng.integers(0, 200))
                    shard_bytes[sh] += rng.integers(0, 256, pad, dtype=np.uint8).tobytes()
                    off = len(shard_bytes[sh])
                    b = np.ascontiguousarray(arr).tobytes()
                    shard_bytes[sh] += b
                    records.append(struct.pack("<iiqq", sh, 0, off, len(b)))
            hm = [P.HostMat(P.DSV4_WFP4, W, S, r, c, 1, 32) for (W, S, r, c) in mats]
            hosts[(L, E)] = P.HostExpert(hm[0], hm[2], hm[1])     # HostExpert(w1, w3, w2)
    for i in reversed(range(n_shards)):
        with open(os.path.join(model_dir, names[i]), "wb") as f:
            f.write(bytes(shard_bytes[i]))
    with open(os.path.join(index_dir, "experts.idx"), "wb") as f:
        f.write(b"DSV4EXP1")
        f.write(struct.pack("<ii", n_layers, n_experts))
        f.write(b"".join(records))
    return model_dir, index_dir, hosts
