"""GPU parity: the 2-D tiled q8_0 / q4_0 GEMM (the panel route for M >= 64,
kernels/quantization/qgemm_panel.cpp:234-286 in the reference) through the
C ABI.

Every row is held to the contract |y - y64| <= 1e-4 * ||x_m||_2 * ||w_n||_2
against the f64 oracle over exactly dequantized weights (all rows for small
shapes, sampled rows at prefill sizes), on both K-range settings and the
automatic route; reruns are bit-identical.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _check(oracle, fmt, packed, x, y, n, k, rows):
    for r in rows:
        y64, wn = oracle.gemv_f64(fmt, packed, x[r], n, k)
        ok, worst = oracle.within_contract(y[r], y64, wn, x[r], TOL)
        assert ok, f"row {r}: normalised error {worst:.3g} > {TOL}"


def _run(qc, dev, fmt, P, x, n, k, mode, x_off=0):
    import torch
    m = x.shape[0]
    X = torch.zeros(m * k + x_off, dtype=torch.float32, device=dev)
    X[x_off:] = torch.from_numpy(x.reshape(-1)).to(dev)
    Y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    qc.set_qgemm_panel(mode)
    try:
        assert qc.qgemm_raw(fmt, P, X[x_off:], Y, m, n, k) == 0
        torch.cuda.synchronize()
    finally:
        qc.set_qgemm_panel(0)
    return Y.cpu().numpy()


@pytest.fixture(params=[1, 2], ids=["one_k_range", "two_k_ranges"])
def split(request):
    return request.param


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m,n,k", [(64, 256, 256), (100, 300, 512), (128, 128, 64),
                                   (130, 1000, 1024), (2, 200, 128), (257, 513, 192),
                                   (129, 255, 4096)])
def test_panel_shapes(qc, oracle, synth, dev, fmt, m, n, k, split):
    import torch
    print(f"panel fmt={fmt} m={m} n={n} k={k} split={split}", flush=True)
    w = synth.normal_fast(31 + n, n * k, 0.02).reshape(n, k)
    st, packed = oracle.pack(fmt, w)
    assert st == 0
    x = synth.normal_fast(37 + m, m * k).reshape(m, k)
    P = torch.from_numpy(packed).to(dev)
    y = _run(qc, dev, fmt, P, x, n, k, split)
    _check(oracle, fmt, packed, x, y, n, k, range(m))
    # bit-identical rerun (two K ranges add onto zero: order-independent)
    assert np.array_equal(y.view(np.uint32), _run(qc, dev, fmt, P, x, n, k, split).view(np.uint32))


@pytest.mark.parametrize("fmt", [0, 1])
def test_panel_activation_range(qc, oracle, synth, dev, fmt):
    """Activations over 40 decades, zero rows, a misaligned x, and a row of
    subnormal activations alone."""
    import torch
    m, n, k = 96, 160, 512
    w = synth.normal_fast(41, n * k, 0.02).reshape(n, k)
    st, packed = oracle.pack(fmt, w)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((m, k)) * 10.0 ** rng.uniform(-20, 20, (m, k))).astype(np.float32)
    x[3] = 0.0
    x[7] = (rng.standard_normal(k) * 1e-39).astype(np.float32)      # subnormal row
    x[9, ::5] = np.float32(3e4)
    P = torch.from_numpy(packed).to(dev)
    for mode, off in ((1, 0), (2, 1), (-1, 0)):
        y = _run(qc, dev, fmt, P, x, n, k, mode, off)
        _check(oracle, fmt, packed, x, y, n, k, range(m))


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m,n,k", [(512, 14336, 4096), (2048, 4096, 4096), (384, 4096, 14336)])
def test_panel_prefill_sizes(qc, oracle, dev, fmt, m, n, k):
    """Prefill shapes of a 4096-hidden / 14336-FFN layer on the automatic
    route (sampled rows; GPU-packed weights are byte-identical to the
    oracle's packer)."""
    import torch
    print(f"panel prefill fmt={fmt} m={m} n={n} k={k}", flush=True)
    g = torch.Generator(device=dev).manual_seed(m + n + k)
    W = torch.randn((n, k), generator=g, device=dev) * 0.02
    P = qc.pack(fmt, W)
    del W
    x = torch.randn((m, k), generator=g, device=dev).cpu().numpy()
    y = _run(qc, dev, fmt, P, x, n, k, 0)
    _check(oracle, fmt, P.cpu().numpy(), x, y, n, k, (0, 1, m // 2, m - 1))
