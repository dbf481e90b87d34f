"""Writes the golden fixtures under tests/golden/ from the reference's own
known answers. Nothing here runs the reference or the oracle: every expected
value is either transcribed from the reference's tests, README or benchmark
log (cited beside it) or known by construction (on-level inputs whose codes
are the inputs themselves, packed by hand with explicit loops).

    python tests/golden/make_golden.py
"""

import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
P = 32


def known_answers() -> dict:
    return {
        "layout_1_5b": {
            "source": "tests/test_quant.py:105-136; README.md:77-82",
            "kv_heads": 2, "head_dim": 128, "page_tokens": 32,
            # The regions in documented order, sizes P*W*bits/8 for each code
            # region, 2W, 2W, 2*P*kv, 2*P*kv for the metadata.
            "metadata_bytes": 1280,
            "effective_bits": {"INT8": 8.625, "INT4": 4.625, "INT2": 2.625},
            "page_bytes": {"FP16": 32768, "INT8": 17664, "INT4": 9472, "INT2": 5376},
            "data_bytes": {"INT8": 16384, "INT4": 8192, "INT2": 4096},
        },
        "footprint_32k_1_5b": {
            "source": "experiments/logs/benchmark.jsonl:48-51 (kv-footprint, measured == computed)",
            "layers": 28, "context": 32768, "granule": 2097152,
            "open_pages_per_layer": {"FP16": 0, "INT8": 2, "INT4": 2, "INT2": 2},
            "bytes": {"FP16": 939524096, "INT8": 509607936, "INT4": 274726912, "INT2": 157286400},
            "payload_bytes": {"FP16": 939524096, "INT8": 508297216, "INT4": 273416192,
                              "INT2": 155975680},
            "effective_bits": {"FP16": 16.0, "INT8": 8.65625, "INT4": 4.65625, "INT2": 2.65625},
        },
        "ewma_first_observation": {
            "source": "tests/test_importance_scores.py:106-115",
            "layers": 2, "max_pages": 8, "layer": 1,
            "mass": [[0.5, 0.25, 0.25], [0.7, 0.2, 0.1]],
            # ((mass[0] + mass[1]) / 2) in fp32, the rest NaN, layer 0 all NaN.
            "expected_first_pages": [0.6, 0.225, 0.175],
        },
        "shapes": {
            "source": "src/microinfer/models.py:18-50 (VERIFIED model cards)",
            "qwen2.5-0.5b": {"layers": 24, "heads": 14, "kv_heads": 2, "head_dim": 64,
                             "hidden": 896, "rope_theta": 1e6, "rms_eps": 1e-6},
            "qwen2.5-1.5b": {"layers": 28, "heads": 12, "kv_heads": 2, "head_dim": 128,
                             "hidden": 1536, "rope_theta": 1e6, "rms_eps": 1e-6},
        },
    }


def hand_pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """8/bits consecutive codes to a byte, the first in the lowest bits
    (quant.h:37-40), one byte at a time."""
    flat = [int(c) for c in codes.reshape(-1)]
    per = 8 // bits
    out = []
    for i in range(0, len(flat), per):
        byte = 0
        for j in range(per):
            byte |= flat[i + j] << (j * bits)
        out.append(byte)
    return np.array(out, np.uint8)


def on_level() -> dict:
    """tests/test_quant.py:181-217: each key channel and value group holds 0
    and 2^bits - 1, so its scale is 1 and zero 0, and its codes are the
    inputs themselves."""
    arrays = {}
    heads, hd = 2, 128
    for name, bits in (("INT8", 8), ("INT4", 4), ("INT2", 2)):
        top = (1 << bits) - 1
        rng = np.random.default_rng(6)
        keys = rng.integers(0, top + 1, (P, heads, hd)).astype(np.float32)
        keys[0], keys[1] = 0, top
        values = rng.integers(0, top + 1, (P, heads, hd)).astype(np.float32)
        values[:, :, 0], values[:, :, 1] = 0, top
        arrays[f"{name}_keys"] = keys
        arrays[f"{name}_values"] = values
        arrays[f"{name}_key_codes"] = hand_pack(keys.astype(np.int64), bits)
        arrays[f"{name}_value_codes"] = hand_pack(values.astype(np.int64), bits)
    return arrays


if __name__ == "__main__":
    (HERE / "known_answers.json").write_text(json.dumps(known_answers(), indent=1) + "\n")
    np.savez_compressed(HERE / "quant_on_level.npz", **on_level())
    print("wrote", HERE / "known_answers.json", HERE / "quant_on_level.npz")
