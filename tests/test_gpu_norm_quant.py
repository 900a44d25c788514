"""GPU parity: rms_norm_add_quant_int8, quantize_int8_asymmetric and
dequantize_int8_asymmetric through the C ABI, bit for bit against the oracle
(itself bit-identical to the reference's compiled functions,
kernels/norms/norm_quant_ref.cpp and kernels/quantization/quantization_ref.cpp).

Every case covers codes, scales, residual_out / zero points and the status;
outputs start as sentinels so that unwritten groups and rows are checked too.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _to(dev, a, off=0):
    """Device copy of a, starting `off` elements into its allocation (off > 0
    breaks 16-byte alignment)."""
    import torch
    a = np.ascontiguousarray(a)
    t = torch.zeros(a.size + off, dtype=getattr(torch, a.dtype.name), device=dev)
    t[off:] = torch.from_numpy(a.reshape(-1)).to(dev)
    return t[off:]


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint8)


def _norm_inputs(seed, rows, hidden, decades=20):
    rng = np.random.default_rng(seed)
    sc = 10.0 ** rng.uniform(-decades, decades)
    x = (rng.standard_normal((rows, hidden)) * sc).astype(np.float32)
    r = (rng.standard_normal((rows, hidden)) * sc).astype(np.float32)
    w = rng.standard_normal(hidden).astype(np.float32)
    return x, r, w


def _norm_gpu(qc, oracle, dev, x, r, w, eps, group, off=0, inplace=None, status=None):
    rows, hidden = x.shape
    g = hidden if group == 0 else group
    X, R, W = _to(dev, x, off), _to(dev, r, off), _to(dev, w, off)
    codes = _to(dev, np.full(rows * hidden, oracle.CODE_SENTINEL, np.int8), off)
    scales = _to(dev, np.full(rows * (hidden // g), oracle.SCALE_SENTINEL, np.float32))
    if inplace == "residual":
        out = R
    elif inplace == "x":
        out = X
    else:
        out = _to(dev, np.zeros(rows * hidden, np.float32), off)
    st = qc.rms_norm_add_quant_int8_raw(X, R, W, codes, out, scales, rows, hidden, eps, group,
                                        status)
    import torch
    torch.cuda.synchronize()
    return (st, codes.cpu().numpy().reshape(rows, hidden), out.cpu().numpy().reshape(rows, hidden),
            scales.cpu().numpy().reshape(rows, hidden // g))


def _norm_check(qc, oracle, dev, x, r, w, eps=1e-5, group=0, **kw):
    want = oracle.rms_norm_add_quant_int8(x, r, w, eps, group)
    got = _norm_gpu(qc, oracle, dev, x, r, w, eps, group, **kw)
    assert got[0] == want[0]
    for g_arr, w_arr, name in zip(got[1:], want[1:], ("codes", "residual_out", "scales")):
        bad = np.argwhere(_bits(g_arr).reshape(g_arr.shape[0], -1) !=
                          _bits(w_arr).reshape(w_arr.shape[0], -1))
        assert bad.size == 0, (name, bad[:5])
    return got


@pytest.fixture(params=[False, True], ids=["settled", "sequential"])
def norm_mode(request, qc):
    qc.set_norm_sequential_sum(request.param)
    yield request.param
    qc.set_norm_sequential_sum(False)


def test_rms_norm_known_answer(qc, oracle, dev, norm_mode):
    # test_remaining_ops.cpp:197-215
    x = np.array([[1, 2, 3, 4]], np.float32)
    got = _norm_check(qc, oracle, dev, x, np.ones((1, 4), np.float32), np.ones(4, np.float32))
    assert list(got[1][0]) == [51, 76, 102, 127] and got[2][0, 3] == 5.0


def test_rms_norm_config3(qc, oracle, dev):
    """The W8A8 producer at BASELINE config 3's shape: 2048 x 4096, per row."""
    print("rms_norm_add_quant 2048x4096", flush=True)
    x, r, w = _norm_inputs(1, 2048, 4096, 2)
    _norm_check(qc, oracle, dev, x, r, w)


@pytest.mark.parametrize("rows,hidden,group", [
    (17, 1000, 0), (5, 1024, 0), (9, 2048, 0), (64, 4096, 32), (33, 4096, 128),
    (16, 4096, 256), (8, 4096, 4), (8, 2048, 8), (8, 1024, 16), (8, 1024, 64),
    (4, 8192, 0), (4, 14336, 0), (3, 16384, 32), (3, 32768, 0),
    # generic kernel: hidden % 4 != 0, > 32768, groups not a power of two or > 256
    (5, 4098, 0), (5, 4098, 2), (2, 40000, 0), (7, 4032, 96), (9, 4096, 512), (3, 6, 3)])
def test_rms_norm_shapes(qc, oracle, dev, norm_mode, rows, hidden, group):
    print(f"rms_norm rows={rows} hidden={hidden} group={group} seq={norm_mode}", flush=True)
    x, r, w = _norm_inputs(rows * 7 + hidden, rows, hidden)
    _norm_check(qc, oracle, dev, x, r, w, 1e-5, group)


@pytest.mark.parametrize("eps", [0.0, 1e-6, 3.0])
@pytest.mark.parametrize("decades", [1, 30])
def test_rms_norm_eps_and_range(qc, oracle, dev, eps, decades):
    x, r, w = _norm_inputs(int(decades * 10 + eps * 7), 6, 4096, decades)
    _norm_check(qc, oracle, dev, x, r, w, eps, 0)
    _norm_check(qc, oracle, dev, x, r, w, eps, 32)


@pytest.mark.parametrize("inplace", ["residual", "x"])
@pytest.mark.parametrize("hidden,group", [(4096, 0), (4096, 64), (4098, 0)])
def test_rms_norm_in_place(qc, oracle, dev, inplace, hidden, group):
    x, r, w = _norm_inputs(hidden + group, 5, hidden)
    _norm_check(qc, oracle, dev, x, r, w, 1e-5, group, inplace=inplace)


@pytest.mark.parametrize("off", [1, 2])
def test_rms_norm_misaligned(qc, oracle, dev, off):
    x, r, w = _norm_inputs(90 + off, 4, 4096)
    _norm_check(qc, oracle, dev, x, r, w, 1e-5, 0, off=off)
    _norm_check(qc, oracle, dev, x, r, w, 1e-5, 32, off=off)


@pytest.mark.parametrize("hidden,group", [(4096, 0), (4096, 32), (4096, 16), (4098, 2),
                                          (4032, 96)])
def test_rms_norm_invalid_groups(qc, oracle, dev, hidden, group):
    """Overflowing and non-finite weights, a NaN input and an all-zero row with
    eps = 0 (0 * inf): those groups keep their sentinels, the call reports 3,
    everything else is written -- synchronously and with a status word."""
    import torch
    x, r, w = _norm_inputs(7, 4, hidden, 1)
    w[5] = np.float32(3e38)
    w[hidden - 40] = np.inf
    x[2, 7] = np.nan
    x[3] = 0.0
    r[3] = 0.0
    for eps in (1e-5, 0.0):
        got = _norm_check(qc, oracle, dev, x, r, w, eps, group)
        assert got[0] == 3
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        got = _norm_gpu(qc, oracle, dev, x, r, w, eps, group, status=status)
        want = oracle.rms_norm_add_quant_int8(x, r, w, eps, group)
        assert got[0] == 0 and int(status.item()) == 3
        for g_arr, w_arr in zip(got[1:], want[1:]):
            assert np.array_equal(_bits(g_arr), _bits(w_arr))


def test_rms_norm_validation(qc, dev):
    import torch
    t = torch.zeros(64, dtype=torch.float32, device=dev)
    c = torch.zeros(64, dtype=torch.int8, device=dev)
    # kernels/norms/norm_quant_ref.cpp:106-130: shape (eps, group), then nulls
    assert qc.rms_norm_add_quant_int8_raw(t, t, t, c, t, t, 2, 32, 1e-5, 5) == 1
    assert qc.rms_norm_add_quant_int8_raw(t, t, t, c, t, t, 2, 32, -1.0, 0) == 1
    assert qc.rms_norm_add_quant_int8_raw(None, t, t, c, t, t, 2, 32, 1e-5, 0) == 3


# ------------------------------------------------ asymmetric int8 ---

def _asym_gpu(qc, dev, x, off=0, status=None):
    import torch
    rows, dim = x.shape
    X = _to(dev, x, off)
    codes = _to(dev, np.full(rows * dim, 0x5A, np.int8), off)
    scales = _to(dev, np.full(rows, -7.0, np.float32))
    zps = _to(dev, np.full(rows, 12345, np.int32))
    st = qc.quantize_int8_asymmetric_raw(X, codes, scales, zps, rows, dim, status)
    torch.cuda.synchronize()
    return st, codes.cpu().numpy().reshape(rows, dim), scales.cpu().numpy(), zps.cpu().numpy()


def _asym_check(qc, oracle, dev, x, off=0):
    want = oracle.quantize_int8_asymmetric(x)
    got = _asym_gpu(qc, dev, x, off)
    assert got[0] == want[0] == 0
    for g_arr, w_arr, name in zip(got[1:], want[1:], ("codes", "scales", "zero_points")):
        assert np.array_equal(_bits(g_arr), _bits(w_arr)), name
    # dequantize, bit for bit
    import torch
    rows, dim = x.shape
    out = torch.empty(rows * dim, dtype=torch.float32, device=dev)
    assert qc.dequantize_int8_asymmetric_raw(_to(dev, want[1]), _to(dev, want[2]),
                                             _to(dev, want[3]), out, rows, dim) == 0
    st, d = oracle.dequantize_int8_asymmetric(*want[1:])
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(d.reshape(-1)))


def test_asym_config3(qc, oracle, dev):
    print("quantize_int8_asymmetric 2048x4096", flush=True)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((2048, 4096)) * 2.0 + 0.5).astype(np.float32)
    _asym_check(qc, oracle, dev, x)


@pytest.mark.parametrize("rows,dim,off", [(1, 2, 0), (3, 1001, 0), (5, 4096, 1), (4, 64, 0),
                                          (2, 14336, 0), (3, 257, 2)])
def test_asym_shapes(qc, oracle, dev, rows, dim, off):
    rng = np.random.default_rng(rows * 100 + dim)
    x = (rng.standard_normal((rows, dim)) * 10.0 ** rng.uniform(-20, 20)).astype(np.float32)
    _asym_check(qc, oracle, dev, x, off)


def test_asym_edges(qc, oracle, dev):
    """Out-of-range zero points and codes (1-ulp spreads across a binade),
    constant rows, the float extremes, tiny values, signed zeros and exact
    half-integer quotients."""
    fmax = np.finfo(np.float32).max
    rows = [np.array([0.99999994, 1.0] * 32, np.float32),
            np.array([1.0, 1.0000001] * 32, np.float32),
            np.full(64, 2.54, np.float32), np.full(64, -1e-12, np.float32),
            np.array([-fmax, fmax] * 32, np.float32),
            np.array([1e-30, 2e-30] * 32, np.float32),
            np.array([0.0, -0.0] * 32, np.float32),
            np.linspace(-3.0, 5.0, 64).astype(np.float32),
            # exact half-integer quotients (scales 1, 2, 1/2, 1/2): ties to even
            np.array([0.0, 255.0] + [k + 0.5 for k in range(62)], np.float32),
            np.array([0.0, 510.0] + [2 * k + 1 for k in range(62)], np.float32),
            np.array([-127.5, 0.0] + [-(k + 0.5) / 2 for k in range(62)], np.float32),
            np.array([-64.0, 63.5] + [(k - 31) * 0.75 for k in range(62)], np.float32)]
    _asym_check(qc, oracle, dev, np.stack(rows))


@pytest.mark.parametrize("off", [0, 1])    # 1: misaligned x, the generic kernel
def test_asym_large_quotients_and_near_ties(qc, oracle, dev, off):
    """Rows whose quotients x / scale run to ~2^32 (a large offset over a tiny
    spread), quotients within 1e-7 relative of a half-integer, 1-ulp spreads
    over every binade and subnormal rows: the codes are rint of the IEEE
    double quotient even where a product with the reciprocal scale rounds the
    other way."""
    print(f"quantize_int8_asymmetric large quotients / near ties off={off}", flush=True)
    rng = np.random.default_rng(11)
    rows = []
    for _ in range(96):
        base = 10.0 ** rng.uniform(-30, 30) * rng.choice([-1.0, 1.0])
        spread = abs(base) * 10.0 ** rng.uniform(-7.5, 2.0)
        rows.append(base + rng.standard_normal(1024) * spread)
    for _ in range(96):
        s = 10.0 ** rng.uniform(-10, 10)
        k = rng.integers(0, 255, 1022)
        near = (k + 0.5) * s * (1.0 + rng.uniform(-1e-7, 1e-7, 1022))
        rows.append(np.concatenate([[0.0, 255.0 * s], near]))
    for _ in range(64):
        b = np.float32(10.0 ** rng.uniform(-20, 20))
        b1 = np.nextafter(b, np.float32(np.inf))
        rows.append(np.array([b, b1, np.nextafter(b1, np.float32(np.inf)), b1] * 256))
    for _ in range(16):
        # subnormal rows (1 / scale beyond the f32 range), and subnormal values
        # under a normal extreme (quotients 0 .. ~60 of subnormal x)
        rows.append(rng.uniform(0.0, 1.0, 1024) * 1e-39)
        top = 10.0 ** rng.uniform(-37, -35)
        rows.append(np.concatenate([[0.0, top], rng.uniform(0.0, 1.0, 1022) * 1.1e-38]))
        rows.append(np.concatenate([[-top, 0.0], -rng.uniform(0.0, 1.0, 1022) * 1.1e-38]))
    _asym_check(qc, oracle, dev, np.stack(rows).astype(np.float32), off)


def test_asym_nonfinite(qc, dev):
    import torch
    x = np.ones((4, 1024), np.float32)
    x[:, 0] = -1.0
    x[2, 5] = np.nan
    # synchronous reference semantics: status 3, nothing written
    st, c, s, z = _asym_gpu(qc, dev, x)
    assert st == 3 and np.all(c == 0x5A) and np.all(s == -7.0) and np.all(z == 12345)
    # asynchronous: finite rows written, the bad row untouched, status word 3
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    st, c, s, z = _asym_gpu(qc, dev, x, status=status)
    assert st == 0 and int(status.item()) == 3
    assert np.all(c[2] == 0x5A) and s[2] == -7.0 and z[2] == 12345
    assert c[0, 0] == -128 and c[0, 1] == 127
