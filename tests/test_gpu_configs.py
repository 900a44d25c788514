"""GPU parity at every BASELINE.json configuration point, at full size, on the
automatic route (the route bench.py times).

* Config 2 (q8_0 small-batch GEMM, K=4096): M in {4, 8, 16, 32} x N in {4096,
  14336}; every output of every row against the f64 contract oracle
  (|y - y64| <= 1e-4 * ||x||_2 * ||w_hat_row||_2, tests/correctness/
  test_qgemv.cpp:278-303 is the reference's form of it).
* Config 4 (the decoder layer's matmul set: Q/K/V/O 4096 x 4096, gate/up
  4096 -> 14336, down 14336 -> 4096):
  - q4_0 at M=1 and M=8, every output against the same contract;
  - q4_0 at M=512 (the prefill panel route bench.py also times), sampled rows;
  - W8A8 at M=512 and M=2048: the activations quantized per row on the GPU
    (codes and scales bit-exact against the oracle's quantize_int8,
    kernels/quantization/quantization_ref.cpp:143-168), the whole int32
    accumulator matrix against a float64 product (exact: every partial sum is
    an integer below 2^53), and 4096 sampled f32 outputs bit-exact against the
    oracle's epilogue (float(dot) * ws[n]) * as[m]
    (kernels/quantization/int8_gemm_ref.cpp:9-32).
Inputs follow the seeded generator of quixicore_hip.synth with config ids 2
and 4; weights ~N(0, 0.02), activations ~N(0, 1), W8A8 activations with 0.1%
outliers x20.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-4
LAYER = ((4096, 4096), (14336, 4096), (4096, 14336))    # (N, K) of config 4's matmuls


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _contract_all_rows(oracle, fmt, packed, x, Y, n, k, rows=None):
    """Every output of the given activation rows against the f64 contract.
    The weights are dequantized once by the oracle's unpack (bit-exact with
    the reference's, pinned in test_oracle.py) and multiplied in float64."""
    w64 = oracle.unpack(fmt, packed, n, k).astype(np.float64)
    wn = np.sqrt(np.einsum("ij,ij->i", w64, w64))
    rows = range(x.shape[0]) if rows is None else rows
    rows = list(rows)
    y64 = x[rows].astype(np.float64) @ w64.T
    worst = 0.0
    for i, r in enumerate(rows):
        ok, wr = oracle.within_contract(Y[r], y64[i], wn, x[r], TOL)
        assert ok, f"row {r}: normalised error {wr:.3g} > {TOL}"
        worst = max(worst, wr)
    return worst


def _packed(oracle, synth, fmt, config, n, k, tensor_id=0):
    st, packed = oracle.pack(fmt, synth.weights(config, n, k, tensor_id=tensor_id))
    assert st == 0
    return packed


@pytest.mark.parametrize("n", [4096, 14336])
@pytest.mark.parametrize("m", [4, 8, 16, 32])
def test_config2_q8_0_small_batch(qc, oracle, synth, dev, m, n):
    """q8_0, K=4096, every (M, N) point, every output."""
    print(f"config2 q8_0 m={m} n={n} k=4096", flush=True)
    k = 4096
    packed = _packed(oracle, synth, 0, 2, n, k)
    x = synth.activations(2, m, k)
    Y = qc.qgemm(0, _t(packed, dev), _t(x, dev), n, k).cpu().numpy()
    worst = _contract_all_rows(oracle, 0, packed, x, Y, n, k)
    print(f"  worst normalised error {worst:.2e}", flush=True)


@pytest.mark.parametrize("n,k", LAYER)
@pytest.mark.parametrize("m", [1, 8])
def test_config4_q4_0_decode(qc, oracle, synth, dev, m, n, k):
    """BASELINE config 4, q4_0 weights at M=1 (qgemv) and M=8 (qgemm), for
    each matmul shape of the layer, every output."""
    print(f"config4 q4_0 m={m} n={n} k={k}", flush=True)
    packed = _packed(oracle, synth, 1, 4, n, k, tensor_id=n // 4096 + k // 4096)
    x = synth.activations(4, m, k, tensor_id=5)
    P, X = _t(packed, dev), _t(x, dev)
    if m == 1:
        Y = qc.qgemv(1, P, X[0].contiguous(), n, k).cpu().numpy().reshape(1, n)
    else:
        Y = qc.qgemm(1, P, X, n, k).cpu().numpy()
    worst = _contract_all_rows(oracle, 1, packed, x, Y, n, k)
    print(f"  worst normalised error {worst:.2e}", flush=True)


@pytest.mark.parametrize("n,k", LAYER)
def test_config4_q4_0_prefill_m512(qc, oracle, synth, dev, n, k):
    """The layer's q4_0 matmuls at M=512 (bench.py's prefill sweep; the 2-D
    panel route): rows across every 128-row m-tile, every output of each."""
    print(f"config4 q4_0 m=512 n={n} k={k}", flush=True)
    m = 512
    packed = _packed(oracle, synth, 1, 4, n, k, tensor_id=n // 4096 + k // 4096)
    x = synth.activations(4, m, k, tensor_id=6)
    Y = qc.qgemm(1, _t(packed, dev), _t(x, dev), n, k).cpu().numpy()
    rows = [0, 1, 63, 64, 127, 128, 255, 256, 383, 384, 510, 511]
    worst = _contract_all_rows(oracle, 1, packed, x, Y, n, k, rows)
    print(f"  worst normalised error {worst:.2e}", flush=True)


@pytest.mark.parametrize("m,n,k", [(512, 4096, 4096), (512, 14336, 4096), (512, 4096, 14336),
                                   (2048, 4096, 14336)])
def test_config4_w8a8(qc, oracle, synth, dev, m, n, k):
    """BASELINE config 4, W8A8 at M=512 (every matmul shape) and the M=2048
    down projection (K=14336; the M=2048 K=4096 shapes are config 3's):
    dynamic per-row quantization on the GPU, then the int8 GEMM."""
    import torch
    print(f"config4 w8a8 m={m} n={n} k={k}", flush=True)
    st, wq, ws = oracle.quantize_int8(synth.weights(4, n, k, tensor_id=8 + k // 4096))
    assert st == 0
    ws = ws[:, 0].copy()
    xf = synth.activations_outliers_fast(4, m, k)
    codes, scales = qc.quantize_int8(_t(xf, dev))
    st, xq, as_ = oracle.quantize_int8(xf)
    assert st == 0
    assert np.array_equal(codes.cpu().numpy(), xq)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), as_.view(np.uint32))
    as_ = as_[:, 0].copy()
    wd = _t(wq, dev)
    Y = qc.int8_gemm(wd, codes, _t(ws, dev), scales[:, 0].contiguous()).cpu().numpy()
    rng = np.random.default_rng(m + n + k)
    rows = np.concatenate([rng.integers(0, m, 4064), np.arange(16) % m, m - 1 - np.arange(16)])
    cols = np.concatenate([rng.integers(0, n, 4064), n - 1 - np.arange(16), np.arange(16)])
    acc, want = oracle.int8_gemm_entries(wq, xq, ws, as_, rows, cols)
    assert np.array_equal(Y[rows, cols].view(np.uint32), want.view(np.uint32))
    A = qc.int8_gemm_i32(wd, codes)
    ref = codes.double() @ wd.double().T.contiguous()
    assert torch.equal(A.double(), ref)
    assert np.array_equal(A.cpu().numpy()[rows, cols].astype(np.int64), acc)
