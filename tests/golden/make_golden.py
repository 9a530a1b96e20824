#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from closed forms only.

The reference ships no fixtures or golden vectors for this path, so every
vector here is derived independently of both the CPU oracle and the GPU code:
  q4k_known.npz     hand-built Q4_K super-blocks (ggml layout of
                    kernels/fst_dequant_q4k_kernel.cc) and their values
                    d*sc_j*q - dmin*m_j computed in float64 (exact) and
                    rounded once to float32;
  mxfp4_known.npz   every FP4 code under several e8m0 exponents, value
                    LUT[nib]*2^(e-127), e in {0,255} -> 0 (kernel semantics);
  philox_kat.json   Philox-4x32-10 known-answer vectors published with
                    Random123 (Salmon et al., SC'11);
  accept_planted.npz greedy-acceptance cases whose answer is fixed by
                    construction (planted argmax per row).
Run: python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.helpers import make_q4k_block  # noqa: E402


def f16_bits(x):
    return int(np.float16(x).view(np.uint16))


def q4k_cases():
    rng = np.random.default_rng(1234)
    blocks, values = [], []

    def add(d, dmin, sc, m, q):
        d16, m16 = f16_bits(d), f16_bits(dmin)
        blocks.append(make_q4k_block(d16, m16, sc, m, q))
        dd = float(np.uint16(d16).view(np.float16))
        mm = float(np.uint16(m16).view(np.float16))
        j = np.arange(256) // 32
        v = dd * np.asarray(sc, np.float64)[j] * np.asarray(q, np.float64) - mm * np.asarray(m, np.float64)[j]
        values.append(v.astype(np.float32))

    # single-nibble impulses: element i only (probes the lo/hi nibble layout)
    for i in [0, 1, 31, 32, 33, 63, 64, 100, 127, 128, 191, 192, 223, 224, 255]:
        q = np.zeros(256, np.int64)
        q[i] = 15
        add(1.0, 0.0, [1] * 8, [0] * 8, q)
    # scale/min patterns covering the 6-bit packing of j < 4 and j >= 4
    add(1.0, 0.5, list(range(1, 9)), list(range(8, 0, -1)), np.arange(256) % 16)
    add(0.25, 0.125, [63] * 8, [63] * 8, np.full(256, 15))
    add(1.0, 1.0, [0, 63, 1, 62, 32, 31, 16, 48], [63, 0, 62, 1, 31, 32, 48, 16], np.arange(256) % 16)
    # subnormal d / dmin (the reference's fp16 decoders mis-decode these)
    add(np.float16(2.0 ** -24), np.float16(3 * 2.0 ** -24), [5] * 8, [7] * 8, np.arange(256) % 16)
    add(np.float16(1023 * 2.0 ** -24), 0.0, [63] * 8, [0] * 8, np.full(256, 15))
    # negative d, zero everything
    add(-0.5, 0.25, [3] * 8, [2] * 8, (np.arange(256) * 7) % 16)
    add(0.0, 0.0, [0] * 8, [0] * 8, np.zeros(256, np.int64))
    # random
    for _ in range(8):
        d = float(np.abs(rng.normal(0, 0.01)))
        dm = float(np.abs(rng.normal(0, 0.01)))
        add(d, dm, rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256))
    return np.stack(blocks), np.stack(values)


def mxfp4_cases():
    lut = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, 0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    blocks, values = [], []
    for e in [0, 1, 100, 119, 127, 128, 140, 254, 255]:
        for start in (0, 8):
            nib = [(start + i) % 16 for i in range(32)]
            blk = np.zeros(17, np.uint8)
            blk[0] = e
            for i in range(16):
                blk[1 + i] = nib[2 * i] | (nib[2 * i + 1] << 4)
            s = 0.0 if e in (0, 255) else 2.0 ** (e - 127)
            blocks.append(blk)
            with np.errstate(over="ignore"):
                values.append(np.array([lut[n] * s for n in nib], np.float32))
    return np.stack(blocks), np.stack(values)


PHILOX_KAT = [
    {"ctr": [0, 0, 0, 0], "key": [0, 0], "out": [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]},
    {"ctr": [0xffffffff] * 4, "key": [0xffffffff] * 2, "out": [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]},
    {"ctr": [0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], "key": [0xa4093822, 0x299f31d0],
     "out": [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]},
]


def accept_cases():
    rng = np.random.default_rng(99)
    k, V = 7, 200
    targets, drafts, n_accs, tokens = [], [], [], []
    for n_acc in range(k + 1):
        t = rng.normal(0, 1, (k + 1, V)).astype(np.float32)
        preds = rng.integers(0, V, k + 1)
        for i in range(k + 1):
            t[i, preds[i]] = 10.0
        draft = preds[:k].copy()
        if n_acc < k:
            draft[n_acc] = (preds[n_acc] + 1) % V
        targets.append(t)
        drafts.append(draft.astype(np.int32))
        n_accs.append(n_acc)
        tok = np.full(k + 1, -1, np.int32)
        tok[:n_acc] = draft[:n_acc]
        tok[n_acc] = preds[n_acc]
        tokens.append(tok)
    return np.stack(targets), np.stack(drafts), np.array(n_accs, np.int32), np.stack(tokens)


def main():
    b, v = q4k_cases()
    np.savez_compressed(os.path.join(HERE, "q4k_known.npz"), blocks=b, values=v)
    b, v = mxfp4_cases()
    np.savez_compressed(os.path.join(HERE, "mxfp4_known.npz"), blocks=b, values=v)
    with open(os.path.join(HERE, "philox_kat.json"), "w") as f:
        json.dump(PHILOX_KAT, f, indent=1)
    t, d, n, tok = accept_cases()
    np.savez_compressed(os.path.join(HERE, "accept_planted.npz"), target=t, draft=d, n_acc=n, tokens=tok)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
