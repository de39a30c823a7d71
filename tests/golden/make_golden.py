"""Writes the golden fixtures of this directory (run from the repository root:
python tests/golden/make_golden.py). Nothing here imports or runs reference code.

gbq_kat.json - the reference's only hand-built known-answer case for the int4
  block layout (tests/ops/_models.py:558-580, gather_block_quantized_model):
  two rows of 32 codes, code k of row r = (k + r) & 15, packed two per byte low
  nibble first, block 16, scales [[0.5, 1], [2, 4]], symmetric (zero point 8),
  gathered with indices [1, -2]. The reference computes its expected output at
  test time with ONNX Runtime; here it is written from the definition of the
  codes (not from the packed bytes), in exact rational arithmetic:
  out[i, k] = ((k + row_i) & 15) - 8) * scale[row_i][k // 16], row_i = idx mod 2.
"""

import json
import os
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))


def gbq_kat():
    rows, codes_per_row, block = 2, 32, 16
    codes = [[(k + r) & 15 for k in range(codes_per_row)] for r in range(rows)]
    packed = [[codes[r][2 * j] | (codes[r][2 * j + 1] << 4) for j in range(codes_per_row // 2)]
              for r in range(rows)]
    scales = [[Fraction(1, 2), Fraction(1)], [Fraction(2), Fraction(4)]]
    indices = [1, -2]
    out = []
    for idx in indices:
        r = idx % rows
        out.append([float((codes[r][k] - 8) * scales[r][k // block]) for k in range(codes_per_row)])
    return {
        "source": "tests/ops/_models.py:558-580 (gather_block_quantized_model)",
        "bits": 4, "block_size": block, "gather_axis": 0, "quantize_axis": 1,
        "data_uint8": packed,
        "indices_int64": indices,
        "scales_f32": [[float(x) for x in row] for row in scales],
        "zero_point": 8,
        "expected_f32": out,
    }


if __name__ == "__main__":
    path = os.path.join(HERE, "gbq_kat.json")
    with open(path, "w") as f:
        json.dump(gbq_kat(), f)
    print("wrote", path)
