"""GPU parity: q8_0 / q4_0 GEMV and small-batch GEMM through the C ABI.

Gate: per output |y - y64| <= 1e-4 * ||x||_2 * ||w_hat_row||_2
against the f64 contract oracle over exactly dequantized weights.  Also bitwise
determinism on rerun, and qgemm row m == qgemv of x[m] within the same gate
(the reference defines qgemm as one qgemv per row,
kernels/quantization/qgemm_ref.cpp:156-162; here M = 1 and M > 1 use different
kernels, so the rows agree to the contract tolerance, not bit for bit).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _case(oracle, synth, fmt, n, k, seed):
    w = synth.normal_fast(seed, n * k, 0.02).reshape(n, k)
    x = synth.normal_fast(seed + 1, k)
    st, packed = oracle.pack(fmt, w)
    assert st == 0
    return packed, x


def _check_rows(oracle, fmt, packed, x, y, n, k):
    y64, wn = oracle.gemv_f64(fmt, packed, x, n, k)
    ok, worst = oracle.within_contract(y, y64, wn, x, TOL)
    assert ok, f"normalised error {worst:.3g} > {TOL}"
    return worst


SHAPES = [(1, 32), (3, 64), (5, 96), (33, 512), (129, 2048), (300, 4096), (64, 14336)]


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("n,k", SHAPES)
def test_qgemv_matches_oracle(qc, oracle, synth, dev, fmt, n, k):
    import torch
    print(f"qgemv fmt={fmt} n={n} k={k}", flush=True)
    packed, x = _case(oracle, synth, fmt, n, k, 1000 + n + k)
    P = torch.from_numpy(packed).to(dev)
    X = torch.from_numpy(x).to(dev)
    y = qc.qgemv(fmt, P, X, n, k)
    y2 = qc.qgemv(fmt, P, X, n, k)
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    _check_rows(oracle, fmt, packed, x, yh, n, k)
    assert np.array_equal(yh.view(np.uint32), y2.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("fmt,n,k", [(0, 4096, 4096), (1, 14336, 4096), (1, 4096, 14336)])
def test_qgemv_baseline_configs(qc, oracle, synth, dev, fmt, n, k):
    """BASELINE configs 0 and 1 at full size, seeded as the bench seeds them."""
    import torch
    print(f"qgemv config fmt={fmt} n={n} k={k}", flush=True)
    cfg = 0 if fmt == 0 else 1
    w = synth.weights(cfg, n, k)
    x = synth.activations(cfg, 1, k)[0]
    st, packed = oracle.pack(fmt, w)
    y = qc.qgemv(fmt, torch.from_numpy(packed).to(dev), torch.from_numpy(x).to(dev), n, k)
    _check_rows(oracle, fmt, packed, x, y.cpu().numpy(), n, k)


@pytest.mark.parametrize("fmt,rows", [(0, 1), (0, 2), (0, 4), (0, 0), (1, 4), (1, 7), (1, 14),
                                      (1, 0)])
def test_whole_line_items(qc, oracle, synth, dev, fmt, rows):
    """Shapes whose GEMV reads each 64-pair item of a row in whole lines and
    restages it through LDS (q8_0 at any row count, q4_0 from 4 rows per
    wave, K <= 4096), beside those that keep per-lane records (K > 4096):
    partial items (K not a multiple of 4096, a last chunk of one pair), rows
    of one pair, a misaligned x, and W allocated to its exact size so the
    last row ends the buffer."""
    import torch
    bb = 34 if fmt == 0 else 18
    qc.set_gemv_rows_per_wave(rows)
    try:
        for n, k in ((1, 64), (7, 192), (65, 2048), (33, 4160), (130, 6144), (9, 8256),
                     (200, 4096)):
            for x_off in (0, 1):
                print(f"whole-line fmt={fmt} rows={rows} n={n} k={k} x_off={x_off}", flush=True)
                packed, x = _case(oracle, synth, fmt, n, k, 4000 + n + k)
                P = torch.from_numpy(packed).to(dev)
                assert P.numel() == n * (k // 32) * bb
                buf = torch.zeros(k + x_off, dtype=torch.float32, device=dev)
                buf[x_off:] = torch.from_numpy(x).to(dev)
                y = qc.qgemv(fmt, P, buf[x_off:], n, k)
                _check_rows(oracle, fmt, packed, x, y.cpu().numpy(), n, k)
    finally:
        qc.set_gemv_rows_per_wave(0)


@pytest.mark.parametrize("rows", [1, 2, 7, 8, 14, 4, 0])
def test_rows_per_wave_variants(qc, oracle, synth, dev, rows):
    import torch
    print(f"rows_per_wave={rows}", flush=True)
    qc.set_gemv_rows_per_wave(rows)
    try:
        for fmt in (0, 1):
            for n, k in ((133, 2048), (70, 8192), (37, 14336), (9, 20480)):
                packed, x = _case(oracle, synth, fmt, n, k, 77)
                y = qc.qgemv(fmt, torch.from_numpy(packed).to(dev), torch.from_numpy(x).to(dev),
                             n, k)
                _check_rows(oracle, fmt, packed, x, y.cpu().numpy(), n, k)
    finally:
        qc.set_gemv_rows_per_wave(0)


@pytest.mark.parametrize("fmt", [0, 1])
def test_qgemv_unaligned_weights(qc, oracle, synth, dev, fmt):
    """Weights at a 2-byte offset take the byte-loading kernel."""
    import torch
    n, k = 40, 1024
    packed, x = _case(oracle, synth, fmt, n, k, 5)
    buf = torch.zeros(packed.size + 2, dtype=torch.uint8, device=dev)
    buf[2:] = torch.from_numpy(packed).to(dev)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    st = qc.qgemv_raw(fmt, buf[2:], torch.from_numpy(x).to(dev), y, n, k)
    assert st == 0
    _check_rows(oracle, fmt, packed, x, y.cpu().numpy(), n, k)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16, 17, 32])
def test_qgemm_small_batch(qc, oracle, synth, dev, fmt, m):
    import torch
    print(f"qgemm fmt={fmt} m={m}", flush=True)
    n, k = 257, 4096
    packed, _ = _case(oracle, synth, fmt, n, k, 31)
    x = synth.normal_fast(4242 + m, m * k).reshape(m, k)
    P = torch.from_numpy(packed).to(dev)
    X = torch.from_numpy(x).to(dev)
    Y = qc.qgemm(fmt, P, X, n, k).cpu().numpy()
    for r in range(m):
        _check_rows(oracle, fmt, packed, x[r], Y[r], n, k)
    # each row is the GEMV of that row (the reference's qgemm definition)
    for r in (0, m - 1):
        yr = qc.qgemv(fmt, P, X[r].contiguous(), n, k).cpu().numpy()
        y64, wn = oracle.gemv_f64(fmt, packed, x[r], n, k)
        ok, worst = oracle.within_contract(yr, Y[r].astype(np.float64), wn, x[r], 2 * TOL)
        assert ok, worst


@pytest.mark.parametrize("fmt,m,n,k", [(0, 33, 300, 192), (1, 40, 129, 64), (0, 5, 2000, 4160),
                                        (1, 32, 4096, 1408), (0, 17, 1000, 14336),
                                        (1, 2, 14336, 4096), (0, 64, 520, 256),
                                        (0, 3, 5, 64), (1, 7, 3, 128), (0, 20, 130, 320),
                                        (1, 4, 14336, 4096), (0, 8, 4096, 4096),
                                        (1, 6, 1000, 14336), (0, 4, 700, 8256),
                                        (1, 9, 260, 4096), (0, 12, 4096, 448),
                                        (0, 10, 300, 8192), (1, 12, 300, 16448)])
def test_qgemm_mfma_shapes(qc, oracle, synth, dev, fmt, m, n, k):
    """Small-batch GEMM shapes that exercise M beyond one 32-row launch,
    partial last K stages, ragged N and split-K partial sums (K up to 16448
    on the f16 / bf16 layouts)."""
    import torch
    print(f"qgemm shapes fmt={fmt} m={m} n={n} k={k}", flush=True)
    packed, _ = _case(oracle, synth, fmt, n, k, 77 + m)
    x = synth.normal_fast(900 + m + k, m * k).reshape(m, k)
    Y = qc.qgemm(fmt, torch.from_numpy(packed).to(dev), torch.from_numpy(x).to(dev), n, k)
    Y = Y.cpu().numpy()
    for r in sorted({0, m // 2, m - 1}):
        _check_rows(oracle, fmt, packed, x[r], Y[r], n, k)
    Y2 = qc.qgemm(fmt, torch.from_numpy(packed).to(dev), torch.from_numpy(x).to(dev), n, k)
    assert np.array_equal(Y2.cpu().numpy().view(np.uint32), Y.view(np.uint32))  # deterministic


@pytest.mark.parametrize("fmt,m", [(0, 3), (1, 7), (1, 12), (0, 20)])
def test_qgemm_every_plan(qc, oracle, synth, dev, fmt, m):
    """Every forced work split (4/8 waves, 1..16 K stages per workgroup, i.e.
    one K range, two atomically added ranges, or partial sums reduced in
    index order) stays within the contract; the digit (m <= 8) and bf16
    activation layouts both."""
    import torch
    n, k = 300, 2304                      # 9 stages: ragged K splits
    packed, _ = _case(oracle, synth, fmt, n, k, 91 + m)
    x = synth.normal_fast(950 + m, m * k).reshape(m, k)
    P, X = torch.from_numpy(packed).to(dev), torch.from_numpy(x).to(dev)
    qc.set_qgemm_rows(-1)               # the MFMA kernels also for m <= 8
    try:
        for waves in (4, 8):
            for stages in (1, 2, 4, 8, 16):
                print(f"qgemm plan fmt={fmt} m={m} waves={waves} stages={stages}", flush=True)
                qc.set_qgemm_plan(waves, stages)
                Y = qc.qgemm(fmt, P, X, n, k).cpu().numpy()
                for r in (0, m - 1):
                    _check_rows(oracle, fmt, packed, x[r], Y[r], n, k)
    finally:
        qc.set_qgemm_plan(0, 0)
        qc.set_qgemm_rows(0)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m,n,k,x_off", [(2, 257, 4096, 0), (3, 4096, 4096, 0),
                                         (4, 14336, 4096, 0), (5, 300, 14336, 0),
                                         (8, 4096, 4096, 0), (7, 1000, 64, 0), (6, 70, 8256, 0),
                                         (8, 130, 4096, 1), (2, 14336, 4096, 3)])
def test_qgemm_rows_bitwise_gemv(qc, oracle, synth, dev, fmt, m, n, k, x_off):
    """The exact-digit rows kernel (forced for every 2 <= M <= 8 here): every
    row of y is bit-identical to qgemv of that activation row (the
    reference's qgemm is one qgemv per row, kernels/quantization/
    qgemm_ref.cpp:156-162), for chunked K (> 4096), ragged N, and x off
    16-byte alignment; the MFMA route for the same shape stays within the
    contract; the automatic route is one of the two."""
    import torch
    print(f"qgemm rows fmt={fmt} m={m} n={n} k={k} x_off={x_off}", flush=True)
    packed, _ = _case(oracle, synth, fmt, n, k, 500 + m)
    x = synth.normal_fast(600 + m + k, m * k).reshape(m, k)
    P = torch.from_numpy(packed).to(dev)
    buf = torch.zeros(m * k + x_off, dtype=torch.float32, device=dev)
    buf[x_off:] = torch.from_numpy(x.reshape(-1)).to(dev)
    X = buf[x_off:].view(m, k)
    Y = torch.empty(m * n, dtype=torch.float32, device=dev)
    for rb in (1, 2, 4):
        qc.set_qgemm_rows(1)
        qc.set_gemv_rows_per_wave(rb)
        try:
            Yr = torch.empty(m * n, dtype=torch.float32, device=dev)
            assert qc.qgemm_raw(fmt, P, X, Yr, m, n, k) == 0
        finally:
            qc.set_qgemm_rows(0)
            qc.set_gemv_rows_per_wave(0)
        if rb > 1:
            assert np.array_equal(Yr.cpu().numpy().view(np.uint32), Y.cpu().numpy().view(np.uint32))
        Y = Yr
    Y = Y.cpu().numpy().reshape(m, n)
    for r in range(m):
        yr = torch.empty(n, dtype=torch.float32, device=dev)
        assert qc.qgemv_raw(fmt, P, X[r], yr, n, k) == 0
        assert np.array_equal(Y[r].view(np.uint32), yr.cpu().numpy().view(np.uint32)), r
    for r in (0, m - 1):
        _check_rows(oracle, fmt, packed, x[r], Y[r], n, k)
    qc.set_qgemm_rows(-1)
    try:
        Y2 = torch.empty(m * n, dtype=torch.float32, device=dev)
        assert qc.qgemm_raw(fmt, P, X, Y2, m, n, k) == 0
        Y2 = Y2.cpu().numpy().reshape(m, n)
    finally:
        qc.set_qgemm_rows(0)
    for r in (0, m - 1):
        _check_rows(oracle, fmt, packed, x[r], Y2[r], n, k)
    Ya = torch.empty(m * n, dtype=torch.float32, device=dev)
    assert qc.qgemm_raw(fmt, P, X, Ya, m, n, k) == 0
    Ya = Ya.cpu().numpy().reshape(m, n).view(np.uint32)
    assert np.array_equal(Ya, Y.view(np.uint32)) or np.array_equal(Ya, Y2.view(np.uint32))


@pytest.mark.parametrize("m,n", [(4, 4096), (32, 14336)])
def test_qgemm_baseline_config2(qc, oracle, synth, dev, m, n):
    """BASELINE config 2 (q8_0, K=4096) at two of its corners."""
    import torch
    print(f"qgemm config2 m={m} n={n}", flush=True)
    k = 4096
    w = synth.weights(2, n, k)
    x = synth.activations(2, m, k)
    st, packed = oracle.pack(0, w)
    Y = qc.qgemm(0, torch.from_numpy(packed).to(dev), torch.from_numpy(x).to(dev), n, k)
    Y = Y.cpu().numpy()
    for r in (0, m // 2, m - 1):
        _check_rows(oracle, 0, packed, x[r], Y[r], n, k)


def test_qgemv_validation_order(qc, dev):
    import torch
    t = torch.zeros(64, dtype=torch.float32, device=dev)
    # src/dispatch/qgemv.cpp:337-349: format, shape, then nulls
    assert qc.qgemv_raw(7, t, t, t, 1, 32) == 2
    assert qc.qgemv_raw(0, t, t, t, 4, 33) == 1
    assert qc.qgemv_raw(0, None, t, t, 1, 32) == 3
    assert qc.qgemm_raw(0, t, t, t, 0, 1, 32) == 1
    assert qc.qgemm_raw(9, None, t, t, 1, 1, 32) == 3  # nulls before format in qgemm


@pytest.mark.parametrize("fmt", [0, 1])
def test_qgemv_adversarial_activations(qc, oracle, synth, dev, fmt):
    """Activations that stress a block-scaled representation: huge and tiny
    values in one block, all-zero blocks, subnormals, 1e30 magnitudes,
    alternating signs and exact ties."""
    import torch
    n, k = 96, 4096
    packed, _ = _case(oracle, synth, fmt, n, k, 505)
    rng = np.random.default_rng(505)
    xs = []
    x = rng.standard_normal(k).astype(np.float32)
    x[::32] *= np.float32(1e6)                    # one giant per block
    xs.append(x)
    x = np.zeros(k, np.float32)
    x[100:164] = rng.standard_normal(64)          # mostly zero blocks
    xs.append(x)
    xs.append((rng.standard_normal(k) * 1e-40).astype(np.float32))   # subnormal
    xs.append((rng.standard_normal(k) * 1e30).astype(np.float32))    # huge
    xs.append(np.where(np.arange(k) % 2 == 0, 1.0, -1.0).astype(np.float32))
    xs.append((np.arange(k) % 255 - 127).astype(np.float32) * np.float32(0.5))
    x = np.exp(rng.uniform(-80, 80, k)).astype(np.float32) * np.sign(rng.standard_normal(k)).astype(np.float32)
    xs.append(x)                                   # 70 decades of dynamic range
    P = torch.from_numpy(packed).to(dev)
    for i, x in enumerate(xs):
        y = qc.qgemv(fmt, P, torch.from_numpy(x).to(dev), n, k).cpu().numpy()
        assert np.all(np.isfinite(y)), i
        worst = _check_rows(oracle, fmt, packed, x, y, n, k)
        print(f"case {i}: worst normalised error {worst:.2e}", flush=True)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m,off", [(12, 1), (32, 0), (25, 3)])
def test_qgemm_dense_activation_range(qc, oracle, synth, dev, fmt, m, off):
    """The bf16 layouts of passes with more than 8 rows: activations over 40
    decades, a zero row, a row of subnormals and one near the float maximum,
    with x at a 4-byte offset from 16-byte alignment (scalar loads in the
    row-exponent and fragment kernel)."""
    import torch
    print(f"qgemm dense range fmt={fmt} m={m} off={off}", flush=True)
    n, k = 200, 1024
    packed, _ = _case(oracle, synth, fmt, n, k, 55 + m)
    rng = np.random.default_rng(m + off)
    x = (rng.standard_normal((m, k)) * 10.0 ** rng.uniform(-20, 20, (m, k))).astype(np.float32)
    x[1] = 0.0
    x[2] = (rng.standard_normal(k) * 1e-40).astype(np.float32)
    x[3] = (rng.standard_normal(k) * 1e37).astype(np.float32)
    X = torch.zeros(m * k + off, dtype=torch.float32, device=dev)
    X[off:] = torch.from_numpy(x.reshape(-1)).to(dev)
    Y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    P = torch.from_numpy(packed).to(dev)
    assert qc.qgemm_raw(fmt, P, X[off:], Y, m, n, k) == 0
    Y = Y.cpu().numpy()
    for r in range(m):
        _check_rows(oracle, fmt, packed, x[r], Y[r], n, k)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m,n,k,waves,stages,x_off", [
    (3, 300, 2304, 4, 1, 0), (4, 14336, 4096, 0, 0, 0), (5, 4096, 4096, 0, 0, 0),
    (8, 4096, 4096, 8, 4, 0), (6, 1000, 14336, 0, 0, 0), (7, 300, 2304, 8, 2, 0),
    (8, 260, 256, 4, 1, 0), (2, 520, 4096, 8, 16, 0), (5, 300, 4096, 4, 8, 3),
    (8, 129, 2304, 4, 8, 0)])
def test_qgemm_fold_bitwise_prep(qc, oracle, synth, dev, fmt, m, n, k, waves, stages, x_off):
    """The digit-layout GEMM that builds its own digits from x (no prep
    launch) gives the same bits as the prep launch + GEMM, for XL = 4 / 8,
    4- and 8-wave workgroups, one K range, two (which keeps the prep launch
    to clear y) and more (partial sums), ragged N, M < XL, and x off 16-byte
    alignment (prep launch); a non-finite activation poisons its row the
    same way in both."""
    import torch
    print(f"qgemm fold fmt={fmt} m={m} n={n} k={k} plan={waves},{stages} x_off={x_off}", flush=True)
    packed, _ = _case(oracle, synth, fmt, n, k, 700 + m)
    x = synth.normal_fast(800 + m + k, m * k).reshape(m, k)
    x[1, 37] = np.inf if m > 2 else x[1, 37]
    P = torch.from_numpy(packed).to(dev)
    buf = torch.zeros(m * k + x_off, dtype=torch.float32, device=dev)
    buf[x_off:] = torch.from_numpy(x.reshape(-1)).to(dev)
    X = buf[x_off:].view(m, k)
    out = {}
    qc.set_qgemm_rows(-1)
    qc.set_qgemm_plan(waves, stages)
    try:
        for fold in (-1, 0):
            qc.set_qgemm_fold(fold)
            Y = torch.full((m * n,), 7.0, dtype=torch.float32, device=dev)
            assert qc.qgemm_raw(fmt, P, X, Y, m, n, k) == 0
            out[fold] = Y.cpu().numpy().reshape(m, n)
    finally:
        qc.set_qgemm_fold(0)
        qc.set_qgemm_plan(0, 0)
        qc.set_qgemm_rows(0)
    assert np.array_equal(out[0].view(np.uint32), out[-1].view(np.uint32))
    for r in (0, m - 1):
        _check_rows(oracle, fmt, packed, x[r], out[0][r], n, k)
    if m > 2:
        assert not np.isfinite(out[0][1]).any()


def _classes(y):
    return np.isnan(y), np.isposinf(y), np.isneginf(y)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("k,x_off", [(4096, 0), (14336, 0), (2048, 1)])
def test_qgemv_nonfinite_activations(qc, oracle, synth, dev, fmt, k, x_off):
    """x holding +-inf or NaN gives each row the reference's f32 result
    class (kernels/quantization/qgemv_ref.cpp:62-80, qgemv_gguf_avx2.cpp:
    295-318: y = sum_b d_b * sum_j q_j x_j): +inf / -inf by the signs of the
    products, NaN where a zero weight meets an infinity, opposite infinities
    meet, or x holds NaN.  The M = 2..4 rows route gives the same bits row
    for row."""
    import torch
    n = 200
    packed, _ = _case(oracle, synth, fmt, n, k, 1200 + k)
    w64 = oracle.unpack(fmt, packed, n, k).astype(np.float64)
    rng = np.random.default_rng(k + fmt)
    base = rng.standard_normal(k).astype(np.float32)
    cases = []
    x = base.copy(); x[97] = np.inf; cases.append(x)
    x = base.copy(); x[k - 5] = -np.inf; cases.append(x)                  # last block
    x = base.copy(); x[40] = np.inf; x[k // 2 + 3] = -np.inf; cases.append(x)
    x = base.copy(); x[300] = np.nan; cases.append(x)
    x = base.copy(); x[0:32] = np.inf; cases.append(x)                    # a whole block
    P = torch.from_numpy(packed).to(dev)
    for i, x in enumerate(cases):
        print(f"nonfinite fmt={fmt} k={k} x_off={x_off} case={i}", flush=True)
        buf = torch.zeros(k + x_off, dtype=torch.float32, device=dev)
        buf[x_off:] = torch.from_numpy(x).to(dev)
        X = buf[x_off:]
        y = torch.empty(n, dtype=torch.float32, device=dev)
        assert qc.qgemv_raw(fmt, P, X, y, n, k) == 0
        y = y.cpu().numpy()
        with np.errstate(invalid="ignore", over="ignore"):
            y64 = (w64 * x.astype(np.float64)[None, :]).sum(axis=1)
        for got, want in zip(_classes(y), _classes(y64)):
            assert np.array_equal(got, want), (i, np.flatnonzero(got != want)[:5])
        assert not np.isfinite(y).any()
    # rows route: every row bit-identical to qgemv of that row
    m = 3
    xm = np.stack([cases[0], base, cases[2]]).astype(np.float32)
    buf = torch.zeros(m * k + x_off, dtype=torch.float32, device=dev)
    buf[x_off:] = torch.from_numpy(xm.reshape(-1)).to(dev)
    X = buf[x_off:].view(m, k)
    qc.set_qgemm_rows(1)
    try:
        Y = torch.empty(m * n, dtype=torch.float32, device=dev)
        assert qc.qgemm_raw(fmt, P, X, Y, m, n, k) == 0
    finally:
        qc.set_qgemm_rows(0)
    Y = Y.cpu().numpy().reshape(m, n)
    for r in range(m):
        yr = torch.empty(n, dtype=torch.float32, device=dev)
        assert qc.qgemv_raw(fmt, P, X[r], yr, n, k) == 0
        assert np.array_equal(Y[r].view(np.uint32), yr.cpu().numpy().view(np.uint32)), r
    assert np.all(np.isfinite(Y[1]))


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m,k,n,panel", [
    (3, 4096, 200, 0),      # digit layout, 4 rows
    (4, 4096, 300, -2),     # digit layout, K split in two (q8_0: both ranges in one workgroup)
    (6, 4096, 4096, 0),     # digit layout, 8 rows, K split four ways
    (8, 14336, 1000, 0),    # digit layout, long K
    (16, 4096, 200, 0),     # f16 / bf16 layout
    (32, 2048, 4096, 0),    # f16 / bf16 layout, 32 rows
    (70, 2048, 300, 1),     # 2-D panel GEMM, one K range
    (70, 4096, 300, 2),     # 2-D panel GEMM, two K ranges (atomic halves)
])
def test_qgemm_mfma_nonfinite_activations(qc, oracle, synth, dev, fmt, m, k, n, panel):
    """The MFMA routes (digit, f16 / bf16 and panel layouts, every K split):
    an activation row holding +-inf or NaN gives each output the reference's
    f32 result class (kernels/quantization/qgemm_ref.cpp:156-162 runs the
    row's qgemv; qgemv_ref.cpp:62-80), and the finite rows are bit-identical
    to the same call with the non-finite rows zeroed."""
    import torch
    packed, _ = _case(oracle, synth, fmt, n, k, 1500 + m + k)
    w64 = oracle.unpack(fmt, packed, n, k).astype(np.float64)
    rng = np.random.default_rng(m * 7 + k + fmt)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bad = {0: [(97, np.inf)], m - 1: [(k - 5, -np.inf)],
           m // 2: [(40, np.inf), (k // 2 + 3, -np.inf), (300, np.nan)]}
    if m > 4:
        bad[1] = [(slice(0, 32), np.inf)]
        bad[3] = [(k - 1, np.nan)]
    xb = x.copy()
    for r, items in bad.items():
        for c, v in items:
            xb[r, c] = v
    P = torch.from_numpy(packed).to(dev)

    def run(xa):
        X = torch.from_numpy(xa).to(dev)
        Y = torch.empty((m, n), dtype=torch.float32, device=dev)
        assert qc.qgemm_raw(fmt, P, X, Y, m, n, k) == 0
        return Y.cpu().numpy()

    print(f"qgemm nonfinite fmt={fmt} m={m} k={k} n={n} panel={panel}", flush=True)
    qc.set_qgemm_panel(panel if panel > 0 else -1)
    qc.set_qgemm_rows(-1)
    if panel == -2:
        qc.set_qgemm_plan(4, 8)   # 16 stages in two K ranges
    try:
        y = run(xb)
        xz = xb.copy()
        xz[sorted(bad)] = 0.0
        yz = run(xz)
    finally:
        qc.set_qgemm_panel(0)
        qc.set_qgemm_rows(0)
        qc.set_qgemm_plan(0, 0)
    for r in range(m):
        if r in bad:
            with np.errstate(invalid="ignore", over="ignore"):
                y64 = (w64 * xb[r].astype(np.float64)[None, :]).sum(axis=1)
            for got, want in zip(_classes(y[r]), _classes(y64)):
                assert np.array_equal(got, want), (r, np.flatnonzero(got != want)[:5])
            assert not np.isfinite(y[r]).any(), r
        else:
            assert np.array_equal(y[r].view(np.uint32), yz[r].view(np.uint32)), r
