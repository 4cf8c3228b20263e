"""Writes codec_kat.json: the packed bytes and packed row offsets of the reference codec
fixture (tests/quantized_matrix_test.cu:15-28, codes (index + row + gene) % (max + 1) at
:78-96) for bits 1/2/4/8 and both metadata policies. Bytes are computed here from the
layout rule of format.cuh:39-48 / layout.cuh:106-129 with numpy, independently of the
oracle, which test_oracle.py then checks against this file."""
import json
from pathlib import Path

import numpy as np

ROW_PTR = np.array([0, 4, 7, 10, 12])
COLS = np.array([0, 2, 5, 7, 1, 4, 6, 0, 3, 7, 2, 5])


def main():
    cases = []
    rows = np.repeat(np.arange(4), np.diff(ROW_PTR))
    for bits in (1, 2, 4, 8):
        cpb = 8 // bits
        codes = (np.arange(len(COLS)) + rows + COLS) % (1 << bits)
        counts = np.diff(ROW_PTR)
        starts = np.concatenate([[0], np.cumsum((counts + cpb - 1) // cpb)])
        out = np.zeros(int(starts[-1]), np.int64)
        for i, (r, c) in enumerate(zip(rows, codes)):
            local = i - ROW_PTR[r]
            out[starts[r] + local // cpb] |= int(c) << int((local % cpb) * bits)
        for policy in (1, 2):
            cases.append({"bits": bits, "policy": policy, "codes": codes.tolist(),
                          "packed_row_ptr": starts.tolist(), "packed": out.tolist()})
    Path(__file__).with_name("codec_kat.json").write_text(json.dumps({"cases": cases}, indent=1))


if __name__ == "__main__":
    main()
