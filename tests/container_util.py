"""Writer of small synthetic apus model containers for the expert-loader tests.

Format (the reference's c/st.h:5-10 and tools/convert.py): each shard is an
8-byte little-endian header length, a JSON header {name: {"dtype", "shape",
"data_offsets": [a, b]}} (offsets relative to the end of the header), then
the payloads back to back; model.safetensors.index.json maps every tensor to
its shard under "weight_map". A routed expert's six tensors
(w1.weight, w1.scale, w2.weight, w2.scale, w3.weight, w3.scale: I8 packed
E2M1 [O, K/2] and F8_E8M0 scales [O, K/32]) form one contiguous slab.
"""
import json
import os
import struct

import numpy as np

MEMBERS = ("w1.weight", "w1.scale", "w2.weight", "w2.scale", "w3.weight", "w3.scale")


def expert_arrays(rng, dim, inter):
    """The six tensors of one expert (uint8): random nibbles, E8M0 118..130."""
    def fp4(O, K):
        return (rng.integers(0, 256, (O, K // 2), dtype=np.uint8),
                rng.integers(118, 131, (O, K // 32), dtype=np.uint8))
    w1, w1s = fp4(inter, dim)
    w2, w2s = fp4(dim, inter)
    w3, w3s = fp4(inter, dim)
    return (w1, w1s, w2, w2s, w3, w3s)


def expert_name(layer, eid, member, mtp=False):
    return f"{'mtp' if mtp else 'layers'}.{layer}.ffn.experts.{eid}.{member}"


def expert_entries(layer, eid, arrays, mtp=False, order=range(6)):
    """(name, dtype, shape, bytes) of one expert's slab, members in `order`."""
    out = []
    for j in order:
        a = arrays[j]
        dt = "F8_E8M0" if j % 2 else "I8"
        out.append((expert_name(layer, eid, MEMBERS[j], mtp), dt, list(a.shape), a.tobytes()))
    return out


def write_shard(path, entries, metadata=True):
    header, blobs, off = {}, [], 0
    if metadata:
        header["__metadata__"] = {"format": "apus"}
    for name, dt, shape, data in entries:
        header[name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def write_container(root, shards, subdir=False, extra_map=None):
    """shards: {file name: [entries]}. Writes the shards and the index under
    root (or root/weights) and returns the directory the index is in."""
    d = os.path.join(root, "weights") if subdir else root
    os.makedirs(d, exist_ok=True)
    wm = {}
    for fname, entries in shards.items():
        write_shard(os.path.join(d, fname), entries)
        for e in entries:
            wm[e[0]] = fname
    if extra_map:
        wm.update(extra_map)
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": wm}, f)
    return d


def dense_entry(name, rng, nbytes=1000):
    return (name, "BF16", [nbytes // 2], rng.integers(0, 256, nbytes, dtype=np.uint8).tobytes())
