"""GPU parity: W8A8 int8 GEMM -- exact int32 accumulators and bit-exact f32
epilogue y = (float(dot) * ws[n]) * as[m] against the oracle, over the
reference's own test grid, BASELINE config 3 and the composed dynamic-W8A8
pipeline (quantize_int8 -> int8 GEMM)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _grid_case(m, n, k, asym, state):
    from test_oracle import _ref_grid_case
    return _ref_grid_case(m, n, k, asym, state)


def test_reference_grid_bit_exact(qc, oracle, dev):
    # tests/correctness/test_int8_gemm.cpp:106-116 (M, N in 1..5, K list, -128, AZP)
    state = [0x9E3779B9]
    for m in range(1, 6):
        for n in range(1, 6):
            for k in (1, 15, 16, 17, 63, 64, 65, 100, 1408):
                for asym in (False, True):
                    w, x, ws, as_, rs, zp = _grid_case(m, n, k, asym, state)
                    st, want = oracle.int8_gemm(w, x, ws, as_, rs, zp, asym)
                    y = qc.int8_gemm(_t(w, dev), _t(x, dev), _t(ws, dev), _t(as_, dev),
                                     _t(rs, dev) if asym else None,
                                     _t(zp, dev) if asym else None, asym)
                    got = y.cpu().numpy()
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, n, k, asym)


@pytest.fixture(params=[0, 1, 2, 3], ids=["auto", "ring", "dma", "staged"])
def route(request, qc):
    qc.set_int8_gemm_route(request.param)
    yield request.param
    qc.set_int8_gemm_route(0)


@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (200, 136, 1408), (37, 301, 4096),
                                   (256, 512, 4160), (5, 4096, 4096), (257, 129, 64),
                                   (300, 200, 128), (520, 130, 192), (1100, 390, 320),
                                   (64, 96, 32), (513, 257, 96), (260, 140, 4128),
                                   (33, 4100, 160), (1030, 6150, 96), (200, 16400, 64),
                                   (1030, 9990, 96),
                                   # steady-state loops of the deep-K tiles: 128 x 128 with a
                                   # 4-deep ring (M 129..256, wide N) and 256 x 256 with a
                                   # 2-deep ring, 8 whole 128-B K steps plus a ragged 32-B one
                                   (256, 14336, 4096), (1030, 9990, 1056),
                                   # up to 32 rows on a wide N: the 64 x 32 tile with an
                                   # 8-deep ring (ragged K, a single row, ragged N)
                                   (7, 14336, 4096), (32, 12352, 1056), (1, 12288, 160),
                                   (19, 12300, 4128)])
def test_accumulators_exact(qc, dev, route, m, n, k):
    import torch
    print(f"int8 acc route={route} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * n + k)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    x = rng.integers(-128, 128, (m, k), dtype=np.int8)
    w[0, :] = -128
    x[0, :] = -128  # the largest products
    wd, xd = _t(w, dev), _t(x, dev)
    acc = qc.int8_gemm_i32(wd, xd)
    # a float64 product is exact here: every partial sum is an integer below 2^53
    want = xd.double() @ wd.double().T.contiguous()
    assert torch.equal(acc.double(), want)


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("m,n,k", [(300, 200, 4096), (700, 390, 1376), (24, 12300, 1056)])
def test_epilogue_bit_exact(qc, oracle, dev, route, m, n, k, asym):
    """Full f32 epilogue (with and without the zero-point correction) on every
    kernel route, bit-exact against the oracle over the whole matrix."""
    print(f"int8 epilogue route={route} m={m} n={n} k={k} asym={asym}", flush=True)
    rng = np.random.default_rng(m + n + k)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    x = rng.integers(-128, 128, (m, k), dtype=np.int8)
    ws = rng.uniform(1e-4, 1e-2, n).astype(np.float32)
    as_ = rng.uniform(1e-3, 1e-1, m).astype(np.float32)
    rs = w.astype(np.int32).sum(axis=1).astype(np.int32) if asym else None
    zp = rng.integers(-128, 128, m).astype(np.int32) if asym else None
    st, want = oracle.int8_gemm(w, x, ws, as_, rs, zp, asym)
    y = qc.int8_gemm(_t(w, dev), _t(x, dev), _t(ws, dev), _t(as_, dev),
                     _t(rs, dev) if asym else None, _t(zp, dev) if asym else None, asym)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("asym", [False, True])
def test_epilogue_deep_tile_rows(qc, oracle, dev, route, asym):
    """The 256 x 256 two-stage tile (M=1030, N=9990, K=1056: 8 whole K steps and a
    ragged one), bit-exact against the oracle on rows that straddle every
    m-tile boundary, over all N columns."""
    print(f"int8 epilogue deep tile route={route} asym={asym}", flush=True)
    m, n, k = 1030, 9990, 1056
    rng = np.random.default_rng(1056 + asym)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    x = rng.integers(-128, 128, (m, k), dtype=np.int8)
    ws = rng.uniform(1e-4, 1e-2, n).astype(np.float32)
    as_ = rng.uniform(1e-3, 1e-1, m).astype(np.float32)
    rs = w.astype(np.int32).sum(axis=1).astype(np.int32) if asym else None
    zp = rng.integers(-128, 128, m).astype(np.int32) if asym else None
    y = qc.int8_gemm(_t(w, dev), _t(x, dev), _t(ws, dev), _t(as_, dev),
                     _t(rs, dev) if asym else None, _t(zp, dev) if asym else None,
                     asym).cpu().numpy()
    rows = np.array([0, 1, 31, 32, 127, 128, 255, 256, 511, 512, 767, 768, 1023, 1024, 1029])
    st, want = oracle.int8_gemm(w, x[rows], ws, as_[rows], rs,
                                zp[rows] if asym else None, asym)
    assert st == 0
    assert np.array_equal(y[rows].view(np.uint32), want.view(np.uint32))


def test_config3_sampled_bit_exact(qc, oracle, synth, dev):
    """BASELINE config 3 (M=2048, K=4096, N=4096): full-size run, 4096 sampled
    outputs bit-exact, plus whole-matrix int32 accumulators vs a float64 BLAS
    product (exact: every partial sum is an integer below 2^53)."""
    import torch
    print("int8 config3 M=2048 N=4096 K=4096", flush=True)
    m, n, k = 2048, 4096, 4096
    wf = synth.weights(3, n, k, tensor_id=3)
    st, wq, ws = oracle.quantize_int8(wf)            # per-output-channel int8 weights
    ws = ws[:, 0].copy()
    x = synth.activations_outliers_fast(3, m, k)
    st, xq, as_ = oracle.quantize_int8(x)
    as_ = as_[:, 0].copy()
    Y = qc.int8_gemm(_t(wq, dev), _t(xq, dev), _t(ws, dev), _t(as_, dev)).cpu().numpy()
    rng = np.random.default_rng(3)
    rows = rng.integers(0, m, 4096)
    cols = rng.integers(0, n, 4096)
    acc, want = oracle.int8_gemm_entries(wq, xq, ws, as_, rows, cols)
    assert np.array_equal(Y[rows, cols].view(np.uint32), want.view(np.uint32))
    A = qc.int8_gemm_i32(_t(wq, dev), _t(xq, dev))
    ref = (torch.from_numpy(xq).to(dev).double() @ torch.from_numpy(wq).to(dev).double().T)
    assert torch.equal(A.double(), ref)


def test_config3_n14336_bit_exact(qc, oracle, synth, dev):
    """BASELINE config 3 at N=14336 (M=2048, K=4096; also config 4's W8A8
    gate/up shape), which takes the 256 x 256 two-stage ring tile: the whole
    int32 matrix against a float64 product, and 4096 sampled f32 outputs
    bit-exact against the oracle."""
    import torch
    print("int8 config3 M=2048 N=14336 K=4096", flush=True)
    m, n, k = 2048, 14336, 4096
    wf = synth.weights(3, n, k, tensor_id=4)
    st, wq, ws = oracle.quantize_int8(wf)
    ws = ws[:, 0].copy()
    x = synth.activations_outliers_fast(3, m, k)
    st, xq, as_ = oracle.quantize_int8(x)
    as_ = as_[:, 0].copy()
    wd, xd = _t(wq, dev), _t(xq, dev)
    Y = qc.int8_gemm(wd, xd, _t(ws, dev), _t(as_, dev)).cpu().numpy()
    rng = np.random.default_rng(14336)
    rows = rng.integers(0, m, 4096)
    cols = rng.integers(0, n, 4096)
    acc, want = oracle.int8_gemm_entries(wq, xq, ws, as_, rows, cols)
    assert np.array_equal(Y[rows, cols].view(np.uint32), want.view(np.uint32))
    A = qc.int8_gemm_i32(wd, xd)
    ref = xd.double() @ wd.double().T.contiguous()
    assert torch.equal(A.double(), ref)


def test_dynamic_w8a8_pipeline(qc, oracle, synth, dev):
    """quantize_int8 on the GPU feeding the GPU GEMM == oracle composition."""
    print("w8a8 pipeline", flush=True)
    m, n, k = 64, 512, 4096
    x = synth.activations_outliers_fast(3, m, k)
    wf = synth.weights(3, n, k, tensor_id=3)
    st, wq, ws = oracle.quantize_int8(wf)
    ws = ws[:, 0].copy()
    xc, xs = qc.quantize_int8(_t(x, dev))
    y = qc.int8_gemm(_t(wq, dev), xc, _t(ws, dev), xs[:, 0].contiguous()).cpu().numpy()
    st, xq, as_ = oracle.quantize_int8(x)
    st, want = oracle.int8_gemm(wq, xq, ws, as_[:, 0].copy())
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_unaligned_and_odd_k(qc, oracle, dev):
    import torch
    rng = np.random.default_rng(1)
    m, n, k = 9, 13, 100
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    x = rng.integers(-128, 128, (m, k), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, n).astype(np.float32)
    as_ = rng.uniform(0.001, 0.01, m).astype(np.float32)
    st, want = oracle.int8_gemm(w, x, ws, as_)
    buf = torch.zeros(n * k + 1, dtype=torch.int8, device=dev)
    buf[1:] = _t(w.reshape(-1), dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    assert qc.int8_gemm_raw(buf[1:], _t(x, dev), _t(ws, dev), _t(as_, dev), None, None, y,
                            m, n, k) == 0
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_validation_and_nonfinite_scales(qc, dev):
    import torch
    w = torch.ones((2, 64), dtype=torch.int8, device=dev)
    x = torch.ones((1, 64), dtype=torch.int8, device=dev)
    ws = torch.tensor([0.5, float("nan")], device=dev)
    as_ = torch.tensor([2.0], device=dev)
    y = torch.full((1, 2), 5.0, device=dev)
    assert qc.int8_gemm_raw(w, x, ws, as_, None, None, y, 1, 2, 0) == 1
    assert qc.int8_gemm_raw(w, x, ws, as_, None, None, None, 1, 2, 64) == 3
    assert qc.int8_gemm_raw(w, x, ws, as_, None, None, y, 1, 2, 64, asymmetric=True) == 3
    assert qc.int8_gemm_raw(w, x, ws, as_, None, None, y, 1, 2, 64) == 3
    assert torch.all(y == 5.0)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    assert qc.int8_gemm_raw(w, x, ws, as_, None, None, y, 1, 2, 64, dev_status=status) == 0
    torch.cuda.synchronize()
    assert int(status.item()) == 3
