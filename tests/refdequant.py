"""Helpers for pinning the oracle against the reference's own C dequantisation
oracles (compiled into oracle/_ref/ from the reference checkout by
oracle/build_ref.py) and against float64 dequantisation.

The C oracles are driven exactly like the reference's tests drive them
(tensor/oracle_q4_k_test.go:161-191): block file in, dense-vector file in,
256 floats + dense dot out.
"""
from __future__ import annotations

import os
import subprocess
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DIR = os.path.join(ROOT, "oracle", "_ref")


def ref_available(name: str) -> bool:
    return os.path.exists(os.path.join(REF_DIR, name))


def run_ref_dequant(name: str, block: bytes, dense=None):
    """Returns (out[256] f32, dense dot f32) from oracle/_ref/<name>."""
    dense = np.ones(256, np.float32) if dense is None else np.asarray(dense, np.float32)
    with tempfile.TemporaryDirectory() as td:
        fin = os.path.join(td, "in.bin")
        fd = os.path.join(td, "dense.bin")
        fo = os.path.join(td, "out.bin")
        with open(fin, "wb") as f:
            f.write(bytes(block))
        dense.astype("<f4").tofile(fd)
        subprocess.run([os.path.join(REF_DIR, name), fin, fd, fo], check=True, capture_output=True)
        raw = np.fromfile(fo, dtype="<f4")
    return raw[:256], raw[256]


def run_ref_q5_0(block: bytes) -> np.ndarray:
    """The 32 floats oracle/_ref/q5_0 writes for one 22-byte block (driven as
    tensor/oracle_c_test.go:104-136 drives it: block file in, floats out)."""
    with tempfile.TemporaryDirectory() as td:
        fin = os.path.join(td, "in.bin")
        fo = os.path.join(td, "out.bin")
        with open(fin, "wb") as f:
            f.write(bytes(block))
        subprocess.run([os.path.join(REF_DIR, "q5_0"), fin, fo], check=True, capture_output=True)
        return np.fromfile(fo, dtype="<f4")[:32]


def dequant_q5_0_f64(blocks: np.ndarray) -> np.ndarray:
    """float64 dequantisation of Q5_0 blocks [n,22] -> [n,32] (layout of
    tensor/oracle_c_test.go:51-72)."""
    blocks = np.asarray(blocks, np.uint8).reshape(-1, 22)
    d = blocks[:, 0:2].copy().view("<f2")[:, 0].astype(np.float64)
    qh = blocks[:, 2:6].copy().view("<u4")[:, 0].astype(np.int64)
    qs = blocks[:, 6:22].astype(np.int64)
    out = np.zeros((len(blocks), 32), np.float64)
    for j in range(16):
        h0 = (qh >> j) & 1
        h1 = (qh >> (j + 16)) & 1
        out[:, j] = d * (((qs[:, j] & 15) | (h0 << 4)) - 16)
        out[:, j + 16] = d * (((qs[:, j] >> 4) | (h1 << 4)) - 16)
    return out


def fp16(b0, b1):
    return np.frombuffer(bytes([b0, b1]), dtype="<f2")[0].astype(np.float64)


def dequant_q4k_f64(blocks: np.ndarray) -> np.ndarray:
    """float64 dequantisation of Q4_K super-blocks [n,144] -> [n,256]
    (layout of the reference's C oracle, tensor/oracle_q4_k_test.go:62-88)."""
    blocks = np.asarray(blocks, np.uint8).reshape(-1, 144)
    n = len(blocks)
    d = blocks[:, 0:2].copy().view("<f2")[:, 0].astype(np.float64)
    dmin = blocks[:, 2:4].copy().view("<f2")[:, 0].astype(np.float64)
    s = blocks[:, 4:16].astype(np.int64)
    sc = np.zeros((n, 8), np.int64)
    m = np.zeros((n, 8), np.int64)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        m[:, j] = s[:, j + 4] & 63
        sc[:, j + 4] = (s[:, j + 8] & 15) | ((s[:, j] >> 6) << 4)
        m[:, j + 4] = (s[:, j + 8] >> 4) | ((s[:, j + 4] >> 6) << 4)
    qs = blocks[:, 16:144].astype(np.int64)
    out = np.zeros((n, 256), np.float64)
    for sb in range(4):
        v = qs[:, sb * 32:(sb + 1) * 32]
        out[:, sb * 64:sb * 64 + 32] = d[:, None] * sc[:, 2 * sb, None] * (v & 15) - dmin[:, None] * m[:, 2 * sb, None]
        out[:, sb * 64 + 32:sb * 64 + 64] = d[:, None] * sc[:, 2 * sb + 1, None] * (v >> 4) - dmin[:, None] * m[:, 2 * sb + 1, None]
    return out


def dequant_q6k_f64(blocks: np.ndarray) -> np.ndarray:
    """float64 dequantisation of Q6_K super-blocks [n,210] -> [n,256]
    (layout of tensor/oracle_q6_k_test.go:62-94)."""
    blocks = np.asarray(blocks, np.uint8).reshape(-1, 210)
    n = len(blocks)
    d = blocks[:, 208:210].copy().view("<f2")[:, 0].astype(np.float64)
    ql = blocks[:, 0:128].astype(np.int64)
    qh = blocks[:, 128:192].astype(np.int64)
    sc = blocks[:, 192:208].view(np.int8).astype(np.int64)
    out = np.zeros((n, 256), np.float64)
    for half in range(2):
        qlN = ql[:, half * 64:(half + 1) * 64]
        qhN = qh[:, half * 32:(half + 1) * 32]
        scN = sc[:, half * 8:(half + 1) * 8]
        for l in range(32):
            is_ = l // 16
            h = qhN[:, l]
            q0 = ((qlN[:, l] & 15) | (((h >> 0) & 3) << 4)) - 32
            q1 = ((qlN[:, l + 32] & 15) | (((h >> 2) & 3) << 4)) - 32
            q2 = ((qlN[:, l] >> 4) | (((h >> 4) & 3) << 4)) - 32
            q3 = ((qlN[:, l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32
            base = half * 128
            out[:, base + l] = d * scN[:, is_] * q0
            out[:, base + l + 32] = d * scN[:, is_ + 2] * q1
            out[:, base + l + 64] = d * scN[:, is_ + 4] * q2
            out[:, base + l + 96] = d * scN[:, is_ + 6] * q3
    return out


def dequant_q8_0_f64(blocks: np.ndarray) -> np.ndarray:
    blocks = np.asarray(blocks, np.uint8).reshape(-1, 34)
    d = blocks[:, 0:2].copy().view("<f2")[:, 0].astype(np.float64)
    q = blocks[:, 2:34].view(np.int8).astype(np.float64)
    return d[:, None] * q


def q8k_dequant_f64(q8k: np.ndarray, nb: int) -> np.ndarray:
    b = np.asarray(q8k, np.uint8)[:nb * 292].reshape(nb, 292)
    d = b[:, 0:4].copy().view("<f4")[:, 0].astype(np.float64)
    q = b[:, 4:260].view(np.int8).astype(np.float64)
    return (d[:, None] * q).reshape(-1)


def q8k_onehot(i: int, nb: int = 1, d: float = 1.0) -> np.ndarray:
    """A Q8_K row with d and a single quant 1 at element i (bsums consistent)."""
    out = np.zeros(nb * 292, np.uint8)
    for b in range(nb):
        out[b * 292:b * 292 + 4] = np.frombuffer(np.float32(d).tobytes(), np.uint8)
    b, e = divmod(i, 256)
    out[b * 292 + 4 + e] = 1
    out[b * 292 + 260 + 2 * (e // 16)] = 1
    return out
