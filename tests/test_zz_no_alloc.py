"""GPU: qc_hip_qgemm_noalloc, the qgemm entry point that allocates nothing
(its scratch is a fixed per-GPU device array), against qc_hip_qgemm through
the C ABI.  Every case makes two no-allocation calls in a row, the second
with a smaller input, so the second reads only what it wrote itself into
the shared array.  Outputs: within the 1e-4 contract bound of the f64
oracle, and equal to qc_hip_qgemm's -- bit for bit where both take the same
plan (passes of <= 32 rows and the same K split), else within the bound.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _problem(oracle, synth, fmt, m, n, k, seed):
    w = synth.normal_fast(seed, n * k, 0.02).reshape(n, k)
    st, packed = oracle.pack(fmt, w)
    assert st == 0
    x = synth.normal_fast(seed + 7, m * k).reshape(m, k)
    return packed, x


def _run_pair(qc, oracle, synth, dev, fmt, first, second, bitwise):
    import torch
    outs = []
    for i, (m, n, k) in enumerate((first, second)):
        print(f"qgemm_noalloc fmt={fmt} call={i} m={m} n={n} k={k}", flush=True)
        packed, x = _problem(oracle, synth, fmt, m, n, k, 4000 + 17 * i + m + n)
        P = torch.from_numpy(packed).to(dev)
        X = torch.from_numpy(x).to(dev)
        y = torch.full((m, n), float("nan"), device=dev)
        st = qc.qgemm_noalloc_raw(fmt, P, X, y, m, n, k)
        assert st == 0, (st, qc.lib.qc_hip_last_error())
        outs.append((packed, x, y, P, X, m, n, k))
    torch.cuda.synchronize()
    for packed, x, y, P, X, m, n, k in outs:
        got = y.cpu().numpy()
        want = qc.qgemm(fmt, P, X, n, k).cpu().numpy()
        y64, wn = oracle.qgemm_f64(fmt, packed, x, n, k)
        for r in range(m):
            ok, worst = oracle.within_contract(got[r], y64[r], wn, x[r], TOL)
            assert ok, ("oracle", m, n, k, r, worst)
            ok, worst = oracle.within_contract(got[r], want[r].astype(np.float64), wn, x[r], TOL)
            assert ok, ("qgemm", m, n, k, r, worst)
        if bitwise:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, n, k)


@pytest.mark.parametrize("fmt", [0, 1])
def test_noalloc_config2_shapes_bitwise(qc, oracle, synth, dev, fmt):
    """Config 2 shapes: digit mode (M=4) after dense tiles (M=32); both entry
    points plan passes with two K ranges here."""
    _run_pair(qc, oracle, synth, dev, fmt, (32, 14336, 4096), (4, 4096, 4096), bitwise=True)


@pytest.mark.parametrize("fmt", [0, 1])
def test_noalloc_dense_then_smaller(qc, oracle, synth, dev, fmt):
    _run_pair(qc, oracle, synth, dev, fmt, (20, 4096, 4096), (9, 1024, 2048), bitwise=False)


@pytest.mark.parametrize("fmt", [0, 1])
def test_noalloc_partials_and_passes(qc, oracle, synth, dev, fmt):
    """K = 12288 needs three K ranges (partial sums in the fixed array);
    then M = 70 runs three passes (qc_hip_qgemm may take the 2-D route)."""
    _run_pair(qc, oracle, synth, dev, fmt, (16, 2048, 12288), (70, 512, 4096), bitwise=False)


def test_noalloc_gemv_and_generic_routes(qc, oracle, synth, dev):
    """M = 1 (the GEMV) and odd K/32 (byte-loading kernel) use no scratch."""
    _run_pair(qc, oracle, synth, dev, 1, (1, 4096, 4096), (3, 100, 96), bitwise=True)


def test_noalloc_rejects_beyond_limits(qc, dev):
    import torch
    k = 16416                                  # above QC_QGEMM_NOALLOC_MAX_K
    P = torch.zeros(2 * (k // 32) * 34, dtype=torch.uint8, device=dev)
    X = torch.zeros((2, k), device=dev)
    y = torch.full((2, 2), 5.0, device=dev)
    assert qc.qgemm_noalloc_raw(0, P, X, y, 2, 2, k) == 1
    assert b"qgemm_noalloc" in qc.lib.qc_hip_last_error()
    # k <= the limit but the K-split partial sums exceed the array:
    # ceil(16384/4096) * 32 * n * 4 bytes with n = 40000 is 20 MB
    k, n = 16384, 40000
    P = torch.zeros(n * (k // 32) * 18, dtype=torch.uint8, device=dev)
    X = torch.zeros((32, k), device=dev)
    y2 = torch.full((32, n), 5.0, device=dev)
    assert qc.qgemm_noalloc_raw(1, P, X, y2, 32, n, k) == 1
    assert b"fixed scratch" in qc.lib.qc_hip_last_error()
    torch.cuda.synchronize()
    assert torch.all(y == 5.0) and torch.all(y2 == 5.0)


def test_noalloc_threads_share_one_stream(qc, oracle, synth, dev):
    """Several host threads calling the no-allocation entry on one stream at
    once: the per-GPU lock queues each call's launch sequence (prep, GEMM,
    reduce) as a whole, so every result is bit-identical to the same call
    made alone, although all calls share the one fixed array."""
    import threading

    import torch
    fmt, n, k = 0, 2048, 4096
    print(f"qgemm_noalloc threads fmt={fmt} n={n} k={k}", flush=True)
    w = synth.normal_fast(91, n * k, 0.02).reshape(n, k)
    st, packed = oracle.pack(fmt, w)
    assert st == 0
    P = torch.from_numpy(packed).to(dev)
    # digit mode (M=4, 6), dense tiles (M=24) and passes of 32 rows (M=40)
    ms = (4, 6, 24, 40)
    xs = {m: synth.normal_fast(990 + m, m * k).reshape(m, k) for m in ms}
    X = {m: torch.from_numpy(xs[m]).to(dev) for m in ms}
    stream = torch.cuda.Stream()          # default priority
    alone = {}
    for m in ms:
        alone[m] = torch.full((m, n), float("nan"), device=dev)
        assert qc.qgemm_noalloc_raw(fmt, P, X[m], alone[m], m, n, k, stream=stream.cuda_stream) == 0
    torch.cuda.synchronize()
    iters = 10
    outs = {m: [torch.full((m, n), float("nan"), device=dev) for _ in range(iters)] for m in ms}
    torch.cuda.synchronize()
    errors = []

    def worker(m):
        try:
            for i in range(iters):
                stt = qc.qgemm_noalloc_raw(fmt, P, X[m], outs[m][i], m, n, k,
                                           stream=stream.cuda_stream)
                if stt != 0:
                    errors.append((m, i, stt))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((m, repr(e)))

    threads = [threading.Thread(target=worker, args=(m,)) for m in ms]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for m in ms:
        want = alone[m].cpu().numpy()
        for i in range(iters):
            got = outs[m][i].cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, i)
        y64, wn = oracle.qgemm_f64(fmt, packed, xs[m], n, k)
        for r in (0, m - 1):
            ok, worst = oracle.within_contract(want[r], y64[r], wn, xs[m][r], TOL)
            assert ok, (m, r, worst)
