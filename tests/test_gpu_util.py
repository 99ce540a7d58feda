"""The measurement kernels of the path (a24): the bandwidth probe's XOR fold against numpy
(bandwidth.comp:1-23) and Context::time_dispatch (skyla-vk/src/submit.rs:31-76), through
the C-ABI."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAGIC = 0x9E3779B9


def _folds(src: np.ndarray, threads: int) -> np.ndarray:
    """Per-thread XOR of the uint4 words src[g], src[g + threads], ... folded to one u32."""
    n = src.shape[0]
    acc = np.zeros((threads, 4), np.uint32)
    for i in range(0, n, threads):
        part = src[i: i + threads]
        acc[: part.shape[0]] ^= part
    return acc[:, 0] ^ acc[:, 1] ^ acc[:, 2] ^ acc[:, 3]


@pytest.mark.parametrize("spec", [[256], [256, 8], [256, 16, 1], [512, 8], [1024, 8, 1]])
@pytest.mark.parametrize("n_vec4", [4096, 4096 + 1000, 37, 3 * 4096 + 4095])
def test_bandwidth_fold_against_numpy(ctx, n_vec4, spec):
    """Every uint4 is folded exactly once, by thread i % (grid x threads), whatever the loads
    in flight per lane: the kernel writes dst[g] only for the threads whose fold is
    0x9e3779b9, and two threads are made so."""
    wg, groups = spec[0], 4
    threads = wg * groups
    g = np.random.default_rng(n_vec4)
    src = g.integers(0, 2**32, size=(n_vec4, 4), dtype=np.uint64).astype(np.uint32)
    f = _folds(src, threads)
    for t in (5, min(n_vec4, threads) - 1):   # patch one word of each to hit the constant
        src[t, 2] ^= np.uint32(f[t] ^ MAGIC)
    want = _folds(src, threads) == MAGIC
    assert want.sum() >= 2
    a = ctx.alloc_host(src.nbytes)
    d = ctx.alloc_host(threads * 4)
    p = ctx.create_pipeline("bandwidth", 2, 4, spec)
    try:
        a.host()[:] = src.reshape(-1).view(np.uint8)
        a.upload()
        d.as_u32()[:] = 0
        d.upload()
        p.bind_buffers([a, d])
        ns = ctx.time_dispatch(p, [groups, 1, 1], [n_vec4], 3)
        d.download()
        got = d.as_u32().copy()
    finally:
        p.free()
        a.free()
        d.free()
    assert np.array_equal(got == MAGIC, want)
    assert np.all(got[~want] == 0)
    assert len(ns) == 3 and all(v > 0 for v in ns)


def test_time_dispatch_reports_each_repetition(ctx):
    """reps timings, each positive and bounded, for a 64 MiB stream read."""
    n_bytes = 64 << 20
    a = ctx.alloc_host(n_bytes)
    d = ctx.alloc_host(1 << 20)
    p = ctx.create_pipeline("bandwidth", 2, 4, [256])
    try:
        p.bind_buffers([a, d])
        ns = ctx.time_dispatch(p, [2048, 1, 1], [n_bytes // 16], 7)
    finally:
        p.free()
        a.free()
        d.free()
    assert len(ns) == 7
    assert all(0 < v < 1e8 for v in ns), ns      # a 64 MiB read takes microseconds, not 0.1 s
    gbs = n_bytes / min(ns)
    assert 100 < gbs < 9000, gbs                 # below the 8 TB/s HBM peak
