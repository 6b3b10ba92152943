"""Writes safetensors shards for the loader tests: an 8-byte little-endian header length,
the JSON header (dtype, shape, data_offsets per tensor, offsets relative to the end of the
header), then the tensors' bytes in the order given."""
import json
import struct

import numpy as np

DT = {np.dtype(np.uint8): "U8", np.dtype(np.float32): "F32", np.dtype(np.uint16): "BF16"}


def write_shard(path, tensors, metadata=None, header_order=None):
    """tensors: [(name, ndarray)] in data order; header_order: the names in the order the
    header lists them (default: data order)."""
    head, off, blobs = {}, 0, []
    for name, a in tensors:
        a = np.ascontiguousarray(a)
        head[name] = {"dtype": DT[a.dtype], "shape": list(a.shape),
                      "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
        blobs.append(a.tobytes())
    if header_order:
        head = {n: head[n] for n in header_order}
    if metadata is not None:
        head = dict({"__metadata__": metadata}, **head)
    hj = json.dumps(head).encode()
    hj += b" " * (-len(hj) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


def expert_name(layer, e, w, kind):
    return f"language_model.model.layers.{layer}.block_sparse_moe.experts.{e}.{w}.{kind}"


def expert_tensors(layer, e, run, geo, inter, hidden):
    """The six tensors of one expert from its run (checkpoint order)."""
    g = geo
    p1 = run[g.p1_off:g.s1_off].reshape(inter, hidden // 2)
    s1 = run[g.s1_off:g.p2_off].reshape(inter, hidden // 32)
    p2 = run[g.p2_off:g.s2_off].reshape(hidden, inter // 2)
    s2 = run[g.s2_off:g.p3_off].reshape(hidden, inter // 32)
    p3 = run[g.p3_off:g.s3_off].reshape(inter, hidden // 2)
    s3 = run[g.s3_off:g.nbytes].reshape(inter, hidden // 32)
    return [(expert_name(layer, e, "w1", "weight_packed"), p1),
            (expert_name(layer, e, "w1", "weight_scale"), s1),
            (expert_name(layer, e, "w2", "weight_packed"), p2),
            (expert_name(layer, e, "w2", "weight_scale"), s2),
            (expert_name(layer, e, "w3", "weight_packed"), p3),
            (expert_name(layer, e, "w3", "weight_scale"), s3)]
