"""Guard bands around device outputs: the device-pointer entry points
(c2h_quantize_q8k_dev, c2h_gemv_dev, c2h_gemv_f32_dev, c2h_logits_ids_dev)
write into caller-allocated device buffers that carry 4 KiB of canary bytes
on each side.  After each call the canaries must be untouched (a kernel
writing past its output would show here rather than as a distant parity
failure), and the output must equal the host-pointer entry point's bit for
bit.  Shapes include ragged row counts and column counts that are not whole
blocks (the reference's floor semantics), where an off-by-one in a grid or
a clamp would write out of bounds."""
import ctypes as C

import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

GUARD = 4096
CANARY = 0xA5


class Guarded:
    """nbytes of device memory between two canary bands (16-byte aligned)."""

    def __init__(self, nbytes: int, fill: bytes | None = None):
        self.nbytes = nbytes
        self.buf = torch.full((2 * GUARD + nbytes,), CANARY, dtype=torch.uint8, device="cuda")
        if fill is not None:
            self.buf[GUARD:GUARD + nbytes] = torch.from_numpy(np.frombuffer(fill, np.uint8).copy()).cuda()
        torch.cuda.synchronize()

    @property
    def ptr(self) -> int:
        return self.buf.data_ptr() + GUARD

    def body(self) -> np.ndarray:
        return self.buf[GUARD:GUARD + self.nbytes].cpu().numpy()

    def check_bands(self):
        head = self.buf[:GUARD].cpu().numpy()
        tail = self.buf[GUARD + self.nbytes:].cpu().numpy()
        assert (head == CANARY).all(), f"{int((head != CANARY).sum())} bytes written before the output"
        assert (tail == CANARY).all(), f"{int((tail != CANARY).sum())} bytes written after the output"


def dev_copy(a: np.ndarray):
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
    torch.cuda.synchronize()
    return t


def call(ctx, name, *args):
    rc = getattr(H.lib(), name)(ctx.h, *args)
    assert rc == H.C2H_OK, (name, rc, H.lib().c2h_last_error(ctx.h))
    assert H.lib().c2h_sync(ctx.h) == H.C2H_OK


@pytest.fixture(scope="module")
def kctx():
    ctx = H.Ctx(None)
    yield ctx
    ctx.close()


@pytest.mark.parametrize("cols", [256, 896, 1000, 4864, 16384])
def test_quantize_q8k_dev_stays_in_bounds(kctx, cols):
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    want = kctx.quantize_q8k(x)
    xd = dev_copy(x)
    out = Guarded(len(want))
    call(kctx, "c2h_quantize_q8k_dev", C.c_void_p(xd.data_ptr()), cols, C.c_void_p(out.ptr))
    out.check_bands()
    assert np.array_equal(out.body(), want)


SYNTH = {H.Q4_K: (G.synth_q4_k, 256, 144), H.Q6_K: (G.synth_q6_k, 256, 210),
         H.Q8_0: (G.synth_q8_0, 32, 34), H.Q5_0: (G.synth_q5_0, 32, 22)}
GEMV_CASES = [(H.Q4_K, 37, 896), (H.Q4_K, 1000, 4864), (H.Q6_K, 37, 896), (H.Q6_K, 999, 4864),
              (H.Q8_0, 37, 896), (H.Q8_0, 151, 1000), (H.Q5_0, 1000, 896)]


def weights(t, rows, cols, seed):
    fn, qk, bs = SYNTH[t]
    return fn(np.random.default_rng(seed), rows * (cols // qk))


@pytest.mark.parametrize("t,rows,cols", GEMV_CASES)
def test_gemv_dev_stays_in_bounds(kctx, t, rows, cols):
    w = weights(t, rows, cols, rows + cols)
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    kquant = t in (H.Q4_K, H.Q6_K)
    if kquant:
        xq = kctx.quantize_q8k(x)
        want, want_is = kctx.gemv(t, w, xq, rows, cols, want_isums=True)
    else:  # the Q8_0 / Q5_0 operator takes the f32 row
        xq = x
        want = kctx.gemv(t, w, x, rows, cols)
    wp = dev_copy(H.pack_weights(t, rows, cols, w))
    xd = dev_copy(xq)
    y = Guarded(rows * 4)
    isums = Guarded(want_is.nbytes) if kquant else None
    call(kctx, "c2h_gemv_dev", t, C.c_void_p(wp.data_ptr()), C.c_void_p(xd.data_ptr()), rows, cols,
         C.c_void_p(y.ptr), C.c_void_p(isums.ptr) if isums else None)
    y.check_bands()
    assert np.array_equal(y.body().view(np.float32), want.view(np.float32))
    if isums:
        isums.check_bands()
        assert np.array_equal(isums.body().view(np.int32), want_is.reshape(-1))


@pytest.mark.parametrize("t,rows,cols", [(H.Q4_K, 37, 896), (H.Q6_K, 1000, 1000), (H.Q8_0, 151, 1000),
                                         (H.Q5_0, 1000, 896), (H.Q4_K, 3, 16384)])
def test_gemv_f32_dev_stays_in_bounds(kctx, t, rows, cols):
    w = weights(t, rows, cols, 3 * rows + cols)
    x = np.random.default_rng(cols + 1).standard_normal(cols).astype(np.float32)
    want = kctx.gemv_f32(t, w, x, rows, cols)
    wp = dev_copy(H.pack_weights(t, rows, cols, w))
    xd = dev_copy(x)
    y = Guarded(rows * 4)
    call(kctx, "c2h_gemv_f32_dev", t, C.c_void_p(wp.data_ptr()), C.c_void_p(xd.data_ptr()), rows, cols,
         C.c_void_p(y.ptr))
    y.check_bands()
    assert np.array_equal(y.body().view(np.float32), want)


def test_logits_ids_dev_stays_in_bounds(tiny_model_path):
    gf = G.GGUFFile(tiny_model_path)
    ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=256))
    H.load_gguf_into(ctx, gf)
    for p, t in enumerate([5, 17, 4095, 300]):
        ctx.forward(t, p, want_normx=False)
    V = ctx.desc.n_vocab
    ids = np.array([0, 7, V - 1, 7, -3, V + 5, 1234], np.int32)  # repeats and out-of-range ids
    base = np.full(V, -7.0, np.float32)
    want = ctx.logits_ids(ids, base.copy())
    idd = dev_copy(ids)
    lg = Guarded(V * 4, fill=base.tobytes())
    call(ctx, "c2h_logits_ids_dev", C.c_void_p(idd.data_ptr()), len(ids), C.c_void_p(lg.ptr))
    lg.check_bands()
    got = lg.body().view(np.float32)
    assert np.array_equal(got, want)
    untouched = np.ones(V, bool)
    untouched[[0, 7, V - 1, 1234]] = False
    assert (got[untouched] == -7.0).all()
    ctx.close()
