"""Writes `.wgpack` files (the reference's prepacked container, src/prepacked/format.ts:118-144)
for tests: synthetic model weights in the tensor names and storages the reference's converter
emits, read back by the package's own parser (js/prepacked.js) in the Node tests."""
import json

import numpy as np

MAGIC = b"WGPACK02"
ALIGN = 256
F32, Q4_0, Q6_K = 0, 2, 14


def _align(x):
    return (x + ALIGN - 1) // ALIGN * ALIGN


def write(path, tensors, metadata=None):
    """tensors: list of (name, dimensions, type, storage, bytes)."""
    table, offset = [], 0
    for name, dims, ttype, storage, data in tensors:
        offset = _align(offset)
        table.append({"name": name, "dimensions": list(dims), "type": ttype, "storage": storage,
                      "offset": offset, "byteLength": len(data)})
        offset += len(data)
    header = {"version": 2, "sourceSha256": "0" * 64, "sourceBytes": 0, "layout": "q4_0-tile32-compact-v2",
              "tileRows": 32, "blockValues": 32, "blockBytes": 20, "metadata": metadata or {}, "tensors": table}
    hb = json.dumps(header).encode()
    start = _align(12 + len(hb))
    out = bytearray(start + offset)
    out[0:8] = MAGIC
    out[8:12] = np.uint32(len(hb)).tobytes()
    out[12:12 + len(hb)] = hb
    for entry, (_, _, _, _, data) in zip(table, tensors):
        out[start + entry["offset"]:start + entry["offset"] + len(data)] = data
    with open(path, "wb") as f:
        f.write(out)


def write_model(path, weights):
    """A model_ref.synthetic_weights() dict as the reference names it (model.ts:86-106)."""
    raw = lambda name, arr, dims, ttype: (name, dims, ttype, "raw", np.ascontiguousarray(arr).tobytes())
    compact = lambda name, t: (name, [t[1], t[2]], Q4_0, "q4_0-tile32-compact", np.asarray(t[0], np.uint8).tobytes())
    tensors = [raw("token_embd.weight", weights["token_embd"], [1024, weights["vocab"]], Q6_K),
               raw("output_norm.weight", weights["output_norm"], [1024], F32)]
    for i, lw in enumerate(weights["layers"]):
        p = f"blk.{i}"
        tensors += [raw(f"{p}.attn_norm.weight", lw["attn_norm"], [1024], F32),
                    compact(f"{p}.attn_qkv.weight", lw["attn_qkv"]),
                    raw(f"{p}.attn_q_norm.weight", lw["attn_q_norm"], [128], F32),
                    raw(f"{p}.attn_k_norm.weight", lw["attn_k_norm"], [128], F32),
                    compact(f"{p}.attn_output.weight", lw["attn_output"]),
                    raw(f"{p}.ffn_norm.weight", lw["ffn_norm"], [1024], F32),
                    compact(f"{p}.ffn_gate_up.weight", lw["ffn_gate_up"]),
                    compact(f"{p}.ffn_down.weight", lw["ffn_down"])]
    write(path, tensors, {"general.architecture": "qwen3", "qwen3.block_count": len(weights["layers"])})
