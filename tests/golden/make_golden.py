"""Writes the golden NF4 dequant fixtures (tests/golden/*.npz) from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its tests compare against bitsandbytes
live, solution/test_nf4.py:12-42), so these fixtures come from the oracle, which is itself
pinned by tests/test_oracle.py.  Each fixture holds the inputs (packed bytes, absmax codes,
code book, second-level scales, offset) and the expected fp16 bit patterns.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def save(name, packed, absmax8, code, absmax2, offset, shape):
    out = O.dequant(packed=packed, absmax8=absmax8, code=code, absmax2=absmax2, offset=offset)
    np.savez_compressed(os.path.join(HERE, f"dequant_{name}.npz"), packed=packed,
                        absmax8=absmax8, code=code, absmax2=absmax2,
                        offset=np.float32(offset), shape=np.array(shape, np.int64),
                        out_bits=out.view(np.uint16).reshape(-1))


def main():
    rng = np.random.default_rng(20240531)
    for shape in [(100, 64), (256, 128)]:
        w = (rng.standard_normal(shape) * 0.02).astype(np.float16)
        q = O.quantize(w)
        save(f"{shape[0]}x{shape[1]}", q.packed, q.absmax8, q.code, q.absmax2, q.offset, shape)
    # edge scales: every byte value under scales that give fp16 subnormals, exact zeros (code 0
    # with zero offset), ordinary values, values that round to the largest finite fp16, and
    # overflow to infinity
    n_blocks = 40
    packed = np.tile(np.arange(256, dtype=np.uint8), n_blocks * 32 // 256)
    code = np.sort(np.concatenate([[0.0], rng.uniform(-1, 1, 254), [1.0]])).astype(np.float32)
    zero = int(np.where(code == 0.0)[0][0])
    absmax8 = rng.integers(0, 256, n_blocks).astype(np.uint8)
    absmax8[:4] = zero
    absmax8[4:8] = 255
    absmax2 = np.array([3e-6], np.float32)  # subnormal fp16 outputs for most blocks
    save("edge_subnormal", packed, absmax8, code, absmax2, 0.0, (n_blocks * 64,))
    save("edge_overflow", packed, absmax8, code, np.array([7e4], np.float32), 1e3,
         (n_blocks * 64,))
    save("edge_ties", packed, absmax8, code, np.array([1.0], np.float32), 0.5, (n_blocks * 64,))


if __name__ == "__main__":
    main()
