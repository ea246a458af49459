"""Writes the golden fixtures of this directory.  Run from the repository root:

    python tests/golden/make_golden.py

Fixtures (all data; nothing here is executed by the tests):

reference_vectors.json
    The vectors the reference's own tests hold for this path, restated as data:
    - binary16 decode KATs: tests/quantization.test.ts:5-9 (`halfToFloat`);
    - the engine's micro-batch packer: tests/embedding-engine.test.ts:5-23 (16 requests coalesce
      into one padded call, results come back in request order) and :25-36 (mixed lengths are
      padded after their final token with the EOS id);
    plus this build's varlen-packing vectors for the same requests (no padding; `cu_seqlens`).

generator_sha256.json
    SHA-256 of the synthetic fp16 Q/K/V arrays (uint16 little-endian bytes, [T, heads*128]) that
    the CPU oracle generates for BASELINE configs 0-4 (config, layer, tensor), and the lengths
    drawn for config 1.  Q and K are after RMSNorm + RoPE.

attention_golden.npz
    The exact (float64 oracle) attention output rounded to fp16 bits for selected rows of each
    config at layer 0, with the row indices and cu_seqlens:
    - cfg0 1x50 full: every row;
    - cfg1 16 ragged (10..150) full: each sequence's last row;
    - cfg2 16x500 full: each sequence's last row;
    - cfg3 1x1500 sparse (176 prefix + 432 window): rows at the mask's boundaries;
    - cfg4 4x5000 sparse: each sequence's middle and last row.
    `cfg0_tiled16_sha256` pins the f16-faithful restatement of the reference's WGSL arithmetic
    on config 0.

MANIFEST.sha256
    SHA-256 of each fixture file.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))

import oracle  # noqa: E402  (test infrastructure: the checker that produces the vectors)

MASK_PREFIX_LOCAL = 1


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).astype("<u2", copy=False).tobytes()).hexdigest()


def cu_of(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def config_lengths(config):
    """Sequence lengths of BASELINE.json configs 0-4."""
    if config == 0:
        return [50]
    if config == 1:
        return oracle.gen_lengths(oracle.seed(1, 0, 3), 16).tolist()
    if config == 2:
        return [500] * 16
    if config == 3:
        return [1500]
    if config == 4:
        return [5000] * 4
    raise ValueError(config)


def golden_rows(config, cu):
    """Token rows whose exact output the fixture keeps."""
    starts, ends = cu[:-1], cu[1:]
    if config == 0:
        return np.arange(int(cu[-1]))
    if config in (1, 2):
        return ends - 1
    if config == 3:
        # first row; last prefix key; first key past the prefix; the window's first full row
        # (432) and its end; the first row whose window leaves the prefix (608); a middle row;
        # the last row
        return np.array([0, 1, 175, 176, 177, 431, 432, 607, 608, 609, 1000, 1499])
    if config == 4:
        return np.stack([starts + (ends - starts) // 2, ends - 1], axis=1).reshape(-1)
    raise ValueError(config)


def reference_vectors():
    return {
        "f16_decode": {
            "source": "tests/quantization.test.ts:5-9",
            "cases": [[0x3C00, 1.0], [0xC000, -2.0], [0x0000, 0.0]],
        },
        "engine_coalesce": {
            "source": "tests/embedding-engine.test.ts:5-23",
            "max_batch": 16,
            "eos": 151643,
            "requests": [[n] for n in range(1, 17)],
            "expect_calls": [{"batch": 16, "sequence": 2, "lengths": [2] * 16}],
            "expect_first_ids": list(range(1, 17)),
        },
        "engine_pad": {
            "source": "tests/embedding-engine.test.ts:25-36",
            "max_batch": 16,
            "eos": 99,
            "requests": [[1], [2, 3]],
            "expect_padded_ids": [1, 99, 99, 2, 3, 99],
        },
        "varlen_pack": {
            "source": "this build: the same requests packed back to back",
            "eos": 99,
            "cases": [
                {"requests": [[1], [2, 3]], "ids": [1, 99, 2, 3, 99], "lengths": [2, 3],
                 "cu_seqlens": [0, 2, 5], "sequence": 3},
                {"requests": [[1], [2, 3], [4, 5, 99]], "ids": [1, 99, 2, 3, 99, 4, 5, 99],
                 "lengths": [2, 3, 3], "cu_seqlens": [0, 2, 5, 8], "sequence": 3},
            ],
        },
    }


def main():
    vectors = reference_vectors()
    with open(os.path.join(HERE, "reference_vectors.json"), "w") as f:
        json.dump(vectors, f, indent=1)
        f.write("\n")

    hashes = {"format": "sha256 of uint16 little-endian fp16 bits, row-major [T, heads*128]",
              "arrays": {}}
    arrays = {}
    for config in range(5):
        lengths = config_lengths(config)
        cu = cu_of(lengths)
        layers = [0, 27] if config >= 2 else [0]
        for layer in layers:
            q, k, v = oracle.gen_qkv(config, layer, cu)
            for name, a in (("q", q), ("k", k), ("v", v)):
                hashes["arrays"][f"cfg{config}/layer{layer}/{name}"] = sha(a)
            if layer != 0:
                continue
            rows = golden_rows(config, cu)
            exact = oracle.attention_exact(q, k, v, cu, MASK_PREFIX_LOCAL, 176, 432, rows=rows)
            arrays[f"cfg{config}_cu"] = cu
            arrays[f"cfg{config}_rows"] = rows.astype(np.int64)
            arrays[f"cfg{config}_out"] = exact.reshape(len(rows), -1).astype(np.float16).view(np.uint16)
            if config == 0:
                tiled = oracle.attention_tiled16(q, k, v, cu)
                arrays["cfg0_tiled16_sha256"] = np.frombuffer(sha(tiled).encode(), dtype=np.uint8)
        if config == 1:
            hashes["cfg1_lengths"] = [int(x) for x in lengths]
    with open(os.path.join(HERE, "generator_sha256.json"), "w") as f:
        json.dump(hashes, f, indent=1)
        f.write("\n")
    np.savez_compressed(os.path.join(HERE, "attention_golden.npz"), **arrays)

    names = ["reference_vectors.json", "generator_sha256.json", "attention_golden.npz"]
    with open(os.path.join(HERE, "MANIFEST.sha256"), "w") as f:
        for n in names:
            with open(os.path.join(HERE, n), "rb") as g:
                f.write(f"{hashlib.sha256(g.read()).hexdigest()}  {n}\n")
    print("wrote", ", ".join(names + ["MANIFEST.sha256"]))


if __name__ == "__main__":
    main()
