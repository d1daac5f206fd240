"""Writes the golden FP8 fixture of tests/golden/.

e4m3fn_bf16_codes.npy: for every bf16 bit pattern u (0..65535) whose value x
is finite, the E4M3FN code of clamp(x, -448, 448) produced by the library
converter ``torch.Tensor.to(torch.float8_e4m3fn)`` (the torch path of
benchmarks/v0/probe_quant_support.py:221-224); non-finite patterns hold 0xFF.
It is produced by torch, not by the oracle, so the oracle is checked against an
independent implementation.

Run: python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.float()
    finite = torch.isfinite(x)
    y = x.clamp(-448.0, 448.0)
    codes = y.to(torch.float8_e4m3fn).view(torch.uint8)
    codes = torch.where(finite, codes, torch.full_like(codes, 0xFF))
    np.save(os.path.join(HERE, "e4m3fn_bf16_codes.npy"), codes.numpy().astype(np.uint8))


if __name__ == "__main__":
    main()
