"""Writes bf16_to_e4m3fn.bin: the E4M3FN code of every bf16 bit pattern.

Source of truth: PyTorch's CPU cast ``Tensor.to(torch.float8_e4m3fn)`` (an
implementation independent of this repository) for every pattern with
|x| <= 448 and for NaN; beyond 448 (where that cast gives NaN) the
reference's saturating conversion defines the code: +-448 (0x7E / 0xFE).
Run:  python tests/golden/make_fp8_lut.py
"""
import hashlib
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def build():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = (bits.astype(np.uint32) << 16).view(np.float32)
    codes = torch.from_numpy(f.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()
    over = ~np.isnan(f) & (np.abs(f) > 448.0)
    codes[over] = np.where(np.signbit(f[over]), 0xFE, 0x7E)
    return codes


if __name__ == "__main__":
    lut = build()
    path = os.path.join(HERE, "bf16_to_e4m3fn.bin")
    lut.tofile(path)
    print(path, hashlib.sha256(lut.tobytes()).hexdigest())
