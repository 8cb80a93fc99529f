"""The C-ABI library loads and exports every entry point include/c2h.h
declares; host-only entry points work without a GPU."""
import ctypes
import os
import re

import numpy as np

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from tests import refdequant as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "c2h.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(c2h_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(H.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_pack_weights_layouts():
    rng = np.random.default_rng(0)
    # Q4_K: the device layout is the reference's own (rows back to back)
    w = G.synth_q4_k(rng, 5 * 3)
    assert np.array_equal(H.pack_weights(H.Q4_K, 5, 896, w), w[:5 * 3 * 144])
    # Q6_K: ql|qh|scales per block, then the fp16 d of every block
    w6 = G.synth_q6_k(rng, 2 * 19)
    p6 = H.pack_weights(H.Q6_K, 2, 4864, w6)
    blocks = w6.reshape(38, 210)
    assert np.array_equal(p6[:38 * 208].reshape(38, 208), blocks[:, :208])
    assert np.array_equal(p6[38 * 208:].reshape(38, 2), blocks[:, 208:])
    # Q8_0: per row 64 bytes of fp16 scales (28 used), then groups of 4 blocks
    # where lane j holds bytes j, j+8, j+16, j+24 of each block
    w8 = G.synth_q8_0(rng, 3 * 28)
    p8 = H.pack_weights(H.Q8_0, 3, 896, w8).reshape(3, 960)
    qs = w8.reshape(3, 28, 34)[:, :, 2:]
    assert np.array_equal(p8[:, :56].reshape(3, 28, 2), w8.reshape(3, 28, 34)[:, :, :2])
    assert not p8[:, 56:64].any()
    q = p8[:, 64:].reshape(3, 7, 8, 4, 4)  # row, group, lane, block-in-group, byte
    for r in range(3):
        for b in range(28):
            for j in range(8):
                for i in range(4):
                    assert q[r, b // 4, j, b % 4, i] == qs[r, b, j + 8 * i]


def test_pack_rejects_bad_shapes():
    w = np.zeros(10, np.uint8)
    out = np.zeros(10, np.uint8)
    L = H.lib()
    assert L.c2h_pack_weights(H.Q4_K, 1, 896, w.ctypes.data, 10, out.ctypes.data, 10) != 0  # short payload
    assert L.c2h_pack_weights(H.Q4_K, 1, 128, w.ctypes.data, 10, out.ctypes.data, 10) != 0  # < 256 cols
    assert L.c2h_pack_weights(3, 1, 896, w.ctypes.data, 10, out.ctypes.data, 10) != 0  # Q4_1 unsupported


def test_row_stride_floor_semantics():
    # tensor/ops.go:121,183: (cols/256)*blockSize -> 896-wide rows cover 3 super-blocks
    assert G.row_bytes(G.Q4_K, 896) == 432
    assert G.row_bytes(G.Q6_K, 896) == 630
    assert G.row_bytes(G.Q4_K, 4864) == 2736
    assert G.row_bytes(G.Q6_K, 4864) == 3990
    assert G.row_bytes(G.Q8_0, 896) == 952
    assert H.packed_size(H.Q4_K, 896, 896) == 896 * 432
