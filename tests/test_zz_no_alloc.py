"""czip_prefill_cdf_noalloc (device buffers in, device buffers out, no
allocation inside) against czip_prefill_cdf on the same inputs, bit for
bit, and on a few chunks against the oracle: two calls in a row, the
second smaller, then the size and token errors.  Device memory for the
inputs and outputs comes from the HIP runtime the library itself links
(ctypes), not from the library."""
import ctypes as C

import numpy as np
import pytest

from conftest import MODEL_PATH

pytestmark = pytest.mark.gpu


class Hip:
    """hipMalloc / hipMemcpy / hipFree of the runtime libczip_hip.so uses."""

    def __init__(self):
        import czip_amd
        czip_amd.lib()  # loads libamdhip64.so.7 first; the same handle is returned below
        self.L = C.CDLL("libamdhip64.so.7")
        self.L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.L.hipFree.argtypes = [C.c_void_p]
        self.L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.L.hipDeviceSynchronize.argtypes = []

    def upload(self, a: np.ndarray) -> int:
        p = C.c_void_p()
        assert self.L.hipMalloc(C.byref(p), max(a.nbytes, 4)) == 0
        assert self.L.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0  # host to device
        return p.value

    def alloc(self, nbytes: int, fill: int = 0xAB) -> int:
        p = self.upload(np.full(nbytes, fill, np.uint8))
        return p

    def download(self, p: int, shape, dtype) -> np.ndarray:
        out = np.zeros(shape, dtype)
        assert self.L.hipDeviceSynchronize() == 0
        assert self.L.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # device to host
        return out

    def free(self, *ps):
        for p in ps:
            self.L.hipFree(p)


@pytest.fixture(scope="module")
def setup():
    import czip_amd
    if czip_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return czip_amd, czip_amd.Model(czip_amd.ModelWeights(MODEL_PATH)), Hip()


def _noalloc(amd, gm, hip, tgt, lens):
    B, T = tgt.shape
    d_t = hip.upload(np.ascontiguousarray(tgt, np.uint32))
    d_l = hip.upload(np.ascontiguousarray(lens, np.int32))
    d_o = hip.alloc(B * T * 8)  # garbage in the output: rows past a length must come back 0
    try:
        rc = amd.lib().czip_prefill_cdf_noalloc(gm._ctx, d_t, d_l, B, T, d_o)
        if rc:
            raise amd.CzipError(rc, amd.lib().czip_last_error(gm._ctx).decode())
        return hip.download(d_o, (B, T, 2), np.uint32)
    finally:
        hip.free(d_t, d_l, d_o)


def _oracle_lohi(om, tgt_row, n):
    """The coder intervals of one chunk's first n targets from the oracle's
    cumulative tables (inputs: BOS 1022, then the targets shifted by one)."""
    inp = np.concatenate([[1022], tgt_row[:n - 1]]).astype(np.uint32)
    _, cum = om.trace(inp)
    t = tgt_row[:n].astype(np.int64)
    lo = np.where(t > 0, cum[np.arange(n), np.maximum(t - 1, 0)], 0)
    return np.stack([lo, cum[np.arange(n), t]], axis=1).astype(np.uint32)


def test_noalloc_equals_prefill_cdf(setup, shipped):
    amd, gm, hip = setup
    rng = np.random.default_rng(120)
    for B, T, lens in [(12, 512, [512, 400, 1, 512, 511, 7, 512, 256, 300, 512, 64, 129]),
                       (3, 100, [100, 37, 0])]:
        print(f"noalloc B={B} T={T}", flush=True)
        tgt = rng.integers(0, 1024, (B, T)).astype(np.uint32)
        got = _noalloc(amd, gm, hip, tgt, lens)
        exp = gm.prefill_cdf(tgt, lens)
        assert np.array_equal(got, exp)
        assert (got[2, lens[2]:] == 0).all()
        # and against the oracle, on a full chunk, a ragged one and a
        # one-token one of the first call
        for b in ([0, 1, 2] if B == 12 else [1]):
            n = lens[b]
            assert np.array_equal(got[b, :n], _oracle_lohi(shipped, tgt[b], n)), f"chunk {b}"


def test_noalloc_limits(setup):
    amd, gm, hip = setup
    with pytest.raises(amd.CzipError) as e:   # ~3.5 KB per row: 64 x 512 rows pass 64 MiB
        _noalloc(amd, gm, hip, np.zeros((64, 512), np.uint32), [512] * 64)
    assert e.value.code == -4
    tgt = np.zeros((2, 64), np.uint32)
    tgt[1, 10] = 5000
    with pytest.raises(amd.CzipError) as e:
        _noalloc(amd, gm, hip, tgt, [64, 64])
    assert e.value.code == -5
    tgt[1, 10] = 0
    tgt[1, 63] = 7000  # past this chunk's length: not read
    assert _noalloc(amd, gm, hip, tgt, [64, 60]).shape == (2, 64, 2)
