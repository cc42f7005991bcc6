"""Write golden vectors for the reference converter's two quantizers.

Runs ONLY in the build container, where the reference tree is mounted:
it imports ``quantize_int8_per_channel`` and ``quantize_int4_per_group`` from
``Scripts/convert_model.py`` (vivekptnk/tinybrain; lines 370-395 and 398-459)
and records their outputs on seeded inputs, including exact rounding ties,
all-zero rows/groups and a ragged last group.  The reference source is not
copied anywhere; only the input/output arrays are kept, in
``converter_vectors.npz`` beside this script.

    python tests/golden/make_converter_vectors.py [/root/reference]
"""
import os
import sys

import numpy as np


def cases():
    rng = np.random.default_rng(20250601)
    out = {}
    # 1. random weights, PyTorch [N, K] layout
    out["rand"] = rng.normal(0.0, 0.02, size=(24, 96)).astype(np.float32)
    # 2. exact ties: absmax 7 (INT4 scale 1.0) / 127 (INT8 scale 1.0)
    t4 = np.array([7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5] * 4, np.float32)
    out["ties4"] = np.stack([t4, -t4, t4 * 0.5 + 0.0]).astype(np.float32)
    t8 = np.array([127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5] * 4, np.float32)
    out["ties8"] = np.stack([t8, -t8]).astype(np.float32)
    # 3. zero rows / zero groups
    z = rng.normal(0.0, 1.0, size=(4, 64)).astype(np.float32)
    z[1, :] = 0.0
    z[2, :32] = 0.0
    out["zeros"] = z
    # 4. ragged: 5 x 7 = 35 elements (odd count, partial last group)
    out["ragged"] = rng.normal(0.0, 3.0, size=(5, 7)).astype(np.float32)
    return out


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, os.path.join(ref, "Scripts"))
    from convert_model import quantize_int4_per_group, quantize_int8_per_channel

    arrays = {}
    for name, w in cases().items():
        arrays[f"{name}__w"] = w
        q8, s8, z8 = quantize_int8_per_channel(w)
        arrays[f"{name}__int8_q"] = np.asarray(q8, np.int8)
        arrays[f"{name}__int8_s"] = np.asarray(s8, np.float32)
        arrays[f"{name}__int8_z"] = np.asarray(z8, np.int8)
        for gs in (32, 64, 128):
            p4, s4, z4 = quantize_int4_per_group(w, group_size=gs)
            arrays[f"{name}__int4_g{gs}_p"] = np.asarray(p4, np.int8)
            arrays[f"{name}__int4_g{gs}_s"] = np.asarray(s4, np.float32)
            arrays[f"{name}__int4_g{gs}_z"] = np.asarray(z4, np.int8)
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "converter_vectors.npz")
    np.savez_compressed(dst, **arrays)
    print(f"wrote {len(arrays)} arrays to {dst}")


if __name__ == "__main__":
    main()
