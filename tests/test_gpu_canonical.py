"""GPU parity: the prepared storage projections over canonical int8 weights
(include/quixicore_cpu/qgemm.h:32-101; kernels/quantization/qgemm_canonical.cpp).

* The scenario list of tests/cpp/storage_scenarios.h runs through this library's
  C++ drop-in with host buffers (tests/cpp/storage_check.cpp) and through the
  reference's own functions (oracle/_ref): every status must be equal, and
  every output of this library must meet the normalised contract against the
  f64 restatement (tests/storage_eval.py), as the reference's own outputs do
  (tests/test_oracle.py).
* The C ABI (qc_hip_cint8_project) at a decoder's shapes: the f32 outputs
  meet the contract; 16-bit outputs are the f32 outputs rounded once (f16:
  IEEE nearest even, bf16: nearest even), bit for bit; 16-bit activations give
  the f32 outputs of their decoded values, bit for bit; the byte-loading route
  (K % 16 != 0, misaligned codes) meets the same contract.
"""
import os
import subprocess

import numpy as np
import pytest

import storage_eval

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "quixicore-cpu_amd", "lib", "storage_check")
TOL = 1e-4


def test_storage_scenarios_match_reference(qc, oracle, ref, tmp_path):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built (make -C quixicore-cpu_amd)")
    ours, theirs = tmp_path / "ours", tmp_path / "ref"
    ours.mkdir()
    theirs.mkdir()
    print("running storage_check", flush=True)
    r = subprocess.run([BINARY, str(ours)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    assert ref.storage_scenarios(theirs) == 0
    status, bad = storage_eval.check(oracle, ours)
    assert not bad, bad[:10]
    ref_status, _ = storage_eval.load(theirs)
    assert status == ref_status


def _bf16_bits(f32):
    b = np.ascontiguousarray(f32, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def _tensor(synth, seed, rows, cols, groups, affine):
    rng = np.random.default_rng(seed)
    codes = rng.integers(-128, 128, (rows, cols), dtype=np.int8)
    scales = (rng.random(rows * groups, dtype=np.float32) * 1e-3 + 1e-5).astype(np.float32)
    zeros = rng.integers(-8, 9, rows * groups).astype(np.float32) if affine else None
    return codes, scales, zeros


def _dev(qc, dev, arr, offset=0):
    import torch
    if arr is None:
        return None
    raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    t = torch.zeros(raw.size + offset, dtype=torch.uint8, device=dev)
    t[offset:] = torch.from_numpy(raw).to(dev)
    return t[offset:]


@pytest.mark.parametrize("rows,cols,groups,affine,m,offset,dot", [
    (14336, 4096, 1, False, 1, 0, 0),     # SmoothQuant-style channel scales, decode
    (14336, 4096, 1, False, 1, 0, -1),    # the same on the f32 multiply-add kernel
    (4096, 4096, 32, True, 1, 0, 0),      # affine, groups of 128
    (4096, 4096, 32, True, 1, 0, -1),
    (1000, 14336, 1, True, 1, 0, 0),      # affine channel scales, K in 4 chunks
    (4096, 14336, 1, False, 1, 0, 0),     # down projection: whole-line code loads, 4 chunks
    (700, 8192, 64, True, 1, 0, 0),       # affine groups of 128, two whole chunks
    (300, 6208, 97, False, 1, 0, 0),      # groups of 64, a last chunk of 33 pairs
    (600, 4096, 128, True, 1, 0, 0),      # groups of 32
    (4096, 14336, 1, False, 2, 0, 1),     # 2-4 rows: digit dots, codes loaded once per pass
    (4096, 14336, 1, False, 3, 0, 0),     # 3 rows: the row-plane route (int8 MFMA)
    (2048, 4096, 32, True, 3, 0, 0),      # affine groups of 128, 3 rows
    (1000, 14336, 1, True, 4, 0, 1),      # affine channel scales, 4 rows, K in 4 chunks
    (1000, 14336, 1, True, 4, 0, 0),      # the same on the row-plane route
    (1000, 14336, 1, True, 4, 0, -1),     # the same on the f32 multiply-add kernel
    (600, 4096, 128, True, 2, 0, 0),      # groups of 32, 2 rows
    (1024, 4096, 64, False, 7, 0, 0),     # passes of 4 activation rows
    (300, 4008, 1, True, 3, 0, 0),        # K % 16 != 0: byte-loading route
    (256, 1024, 4, False, 2, 4, 0),       # misaligned codes: byte-loading route
    (130, 96, 3, True, 5, 0, 0),          # groups of 32 over K = 96
])
def test_cint8_project_contract(qc, oracle, synth, dev, rows, cols, groups, affine, m, offset, dot):
    import torch
    print(f"cint8 rows={rows} cols={cols} groups={groups} affine={affine} m={m} off={offset} "
          f"dot={dot}", flush=True)
    qc.set_cint8_dot(dot)
    try:
        _contract_case(qc, oracle, synth, dev, rows, cols, groups, affine, m, offset)
    finally:
        qc.set_cint8_dot(0)


def _contract_case(qc, oracle, synth, dev, rows, cols, groups, affine, m, offset):
    import torch
    codes, scales, zeros = _tensor(synth, rows + cols, rows, cols, groups, affine)
    x = synth.normal_fast(7 + m, m * cols).reshape(m, cols)
    C = _dev(qc, dev, codes, offset)
    S, Z = _dev(qc, dev, scales), _dev(qc, dev, zeros)
    w = qc.cint8_weights(C, S, Z, rows, cols, groups)
    X = torch.from_numpy(x).to(dev)
    y = torch.empty(m * rows, dtype=torch.float32, device=dev)
    assert qc.cint8_project_raw(0, [w], X, 0, m, [y], [0]) == 0
    yf = y.cpu().numpy().reshape(m, rows)
    what = oracle.cint8_dequant(codes, scales, zeros, rows, cols, groups)
    y64, wn = oracle.cint8_project_f64(x, what)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    assert np.all(np.abs(yf - y64) <= TOL * xn * wn[None, :])
    # 16-bit outputs: the f32 values rounded once
    for name, t, want in (("f16", 1, yf.astype(np.float16).view(np.uint16)),
                          ("bf16", 2, _bf16_bits(yf))):
        h = torch.empty(m * rows, dtype=torch.int16, device=dev)
        assert qc.cint8_project_raw(0, [w], X, 0, m, [h], [t]) == 0
        got = h.cpu().numpy().view(np.uint16).reshape(m, rows)
        assert np.array_equal(got, want.reshape(m, rows)), name
    # 16-bit activations: the f32 outputs of their decoded values
    xb = _bf16_bits(x)
    xd = (xb.astype(np.uint32) << 16).view(np.float32).reshape(m, cols)
    yd = torch.empty(m * rows, dtype=torch.float32, device=dev)
    assert qc.cint8_project_raw(0, [w], torch.from_numpy(xd).to(dev), 0, m, [yd], [0]) == 0
    yb = torch.empty(m * rows, dtype=torch.float32, device=dev)
    XB = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
    assert qc.cint8_project_raw(0, [w], XB, 2, m, [yb], [0]) == 0
    assert np.array_equal(yb.cpu().numpy().view(np.uint32), yd.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("groups,affine,x_type", [(1, False, 0), (1, True, 0), (32, True, 2),
                                                  (32, False, 1)])
def test_cint8_nonfinite_activations(qc, oracle, synth, dev, groups, affine, x_type):
    """One activation row holding +-inf or NaN: every output gets the
    reference's f32 class (decode w = s * (q - z), then sum w x;
    kernels/quantization/qgemm_canonical.cpp:125-176): +-inf by the signs of
    the products, NaN where a zero weight meets an infinity, opposite
    infinities meet, or x holds NaN; on both M = 1 kernels."""
    import torch
    rows, cols = 300, 4096
    codes, scales, zeros = _tensor(synth, 77 + groups, rows, cols, groups, affine)
    codes[:, 200] = 0                                   # zero codes meet the infinity
    if zeros is not None:
        zeros[::5] = 0.0
    keep = [_dev(qc, dev, a) for a in (codes, scales, zeros)]
    w = qc.cint8_weights(keep[0], keep[1], keep[2], rows, cols, groups)
    what = oracle.cint8_dequant(codes, scales, zeros, rows, cols, groups).astype(np.float64)
    rng = np.random.default_rng(groups)
    base = rng.standard_normal(cols).astype(np.float32)
    cases = []
    x = base.copy(); x[200] = np.inf; cases.append(x)
    x = base.copy(); x[77] = -np.inf; x[3000] = np.inf; cases.append(x)
    x = base.copy(); x[1234] = np.nan; cases.append(x)
    x = base.copy(); x[4000] = np.inf; cases.append(x)
    for dot in (0, -1):
        qc.set_cint8_dot(dot)
        try:
            for i, x in enumerate(cases):
                print(f"cint8 nonfinite groups={groups} affine={affine} x_type={x_type} dot={dot} "
                      f"case={i}", flush=True)
                if x_type == 0:
                    X = torch.from_numpy(x).to(dev)
                    xd = x
                elif x_type == 1:
                    xh = x.astype(np.float16)
                    X = torch.from_numpy(xh.view(np.int16).copy()).to(dev)
                    xd = xh.astype(np.float32)
                else:
                    xb = _bf16_bits(x)
                    X = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
                    xd = (xb.astype(np.uint32) << 16).view(np.float32)
                y = torch.empty(rows, dtype=torch.float32, device=dev)
                assert qc.cint8_project_raw(0, [w], X, x_type, 1, [y], [0]) == 0
                y = y.cpu().numpy()
                with np.errstate(invalid="ignore", over="ignore"):
                    y64 = (what * xd.astype(np.float64)[None, :]).sum(axis=1)
                for got, want in ((np.isnan(y), np.isnan(y64)), (np.isposinf(y), np.isposinf(y64)),
                                  (np.isneginf(y), np.isneginf(y64))):
                    assert np.array_equal(got, want), (i, np.flatnonzero(got != want)[:5])
        finally:
            qc.set_cint8_dot(0)


@pytest.mark.parametrize("groups,affine,x_type,m", [(1, False, 0, 2), (1, True, 0, 3), (32, True, 2, 4),
                                                    (32, False, 1, 4)])
def test_cint8_rows_match_one_row(qc, oracle, synth, dev, groups, affine, x_type, m):
    """2-4 activation rows on the digit-dot kernel (forced: row scales would
    take the row-plane route by default): every output row is
    bit-identical to the one-row call on that row (same digits, order and
    finish), finite rows and rows holding +-inf or NaN alike."""
    import torch
    rows, cols = 300, 4096
    codes, scales, zeros = _tensor(synth, 91 + groups, rows, cols, groups, affine)
    codes[:, 200] = 0
    keep = [_dev(qc, dev, a) for a in (codes, scales, zeros)]
    w = qc.cint8_weights(keep[0], keep[1], keep[2], rows, cols, groups)
    rng = np.random.default_rng(m + groups)
    xs = rng.standard_normal((m, cols)).astype(np.float32)
    xs[0, 200] = np.inf
    xs[m - 1, 1234] = np.nan
    if x_type == 0:
        X = torch.from_numpy(xs).to(dev)
    elif x_type == 1:
        X = torch.from_numpy(xs.astype(np.float16).view(np.int16).copy()).to(dev)
    else:
        X = torch.from_numpy(_bf16_bits(xs).view(np.int16).copy()).to(dev)
    print(f"cint8 rows vs one row groups={groups} affine={affine} x_type={x_type} m={m}", flush=True)
    Y = torch.empty((m, rows), dtype=torch.float32, device=dev)
    qc.set_cint8_dot(1)                       # the digit-dot kernels, not the row-plane route
    try:
        assert qc.cint8_project_raw(0, [w], X, x_type, m, [Y], [0]) == 0
    finally:
        qc.set_cint8_dot(0)
    Y = Y.cpu().numpy()
    for r in range(m):
        y1 = torch.empty(rows, dtype=torch.float32, device=dev)
        assert qc.cint8_project_raw(0, [w], X[r].contiguous(), x_type, 1, [y1], [0]) == 0
        assert np.array_equal(Y[r].view(np.uint32), y1.cpu().numpy().view(np.uint32)), r
    assert not np.isfinite(Y[0]).any()
    if m > 2:
        assert np.isfinite(Y[1]).all()


def test_cint8_fused_decode_shapes(qc, oracle, synth, dev):
    """SwiGLU and RoPE Q/K/V at a decoder's shapes: bit-identical to the f32
    epilogue applied to the plain projections of the same launch family."""
    import torch
    cols = 4096
    g_codes, g_s, _ = _tensor(synth, 1, 14336, cols, 1, False)
    u_codes, u_s, _ = _tensor(synth, 2, 14336, cols, 1, False)
    x = synth.normal_fast(3, cols)
    X = torch.from_numpy(x).to(dev)
    keep = [_dev(qc, dev, a) for a in (g_codes, g_s, u_codes, u_s)]   # device buffers stay alive
    G = qc.cint8_weights(keep[0], keep[1], None, 14336, cols, 1)
    U = qc.cint8_weights(keep[2], keep[3], None, 14336, cols, 1)
    gate = torch.empty(14336, dtype=torch.float32, device=dev)
    up = torch.empty(14336, dtype=torch.float32, device=dev)
    out = torch.empty(14336, dtype=torch.float32, device=dev)
    assert qc.cint8_project_raw(0, [G, U], X, 0, 1, [gate, up], [0, 0]) == 0
    assert qc.cint8_project_raw(1, [G, U], X, 0, 1, [out], [0]) == 0
    g, u = gate.cpu().numpy(), up.cpu().numpy()
    gp = torch.empty(14336, dtype=torch.float32, device=dev)
    assert qc.cint8_project_raw(0, [G], X, 0, 1, [gp], [0]) == 0
    assert np.array_equal(gp.cpu().numpy().view(np.uint32), g.view(np.uint32))
    want = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32) * u
    o = out.cpu().numpy()
    assert np.all(np.abs(o - want) <= 4e-7 * np.abs(want) + 1e-30)
    # RoPE: 32 query heads, 8 kv heads of 128
    q_c, q_s, _ = _tensor(synth, 4, 4096, cols, 1, False)
    k_c, k_s, _ = _tensor(synth, 5, 1024, cols, 1, False)
    v_c, v_s, _ = _tensor(synth, 6, 1024, cols, 1, False)
    keep += [_dev(qc, dev, a) for a in (q_c, q_s, k_c, k_s, v_c, v_s)]
    Ws = [qc.cint8_weights(keep[4 + 2 * i], keep[5 + 2 * i], None, c.shape[0], cols, 1)
          for i, c in enumerate((q_c, k_c, v_c))]
    ang = synth.normal_fast(8, 64)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    plain = [torch.empty(r, dtype=torch.float32, device=dev) for r in (4096, 1024, 1024)]
    assert qc.cint8_project_raw(0, Ws, X, 0, 1, plain, [0, 0, 0]) == 0
    rot = [torch.empty(r, dtype=torch.float32, device=dev) for r in (4096, 1024, 1024)]
    assert qc.cint8_project_raw(2, Ws, X, 0, 1, rot, [0, 0, 0], rope_cos=torch.from_numpy(cs).to(dev),
                                rope_sin=torch.from_numpy(sn).to(dev), head_dim=128) == 0
    for i, heads in ((0, 32), (1, 8)):
        p = plain[i].cpu().numpy().reshape(heads, 2, 64)
        a, b = p[:, 0], p[:, 1]
        want = np.stack([a * cs - b * sn, b * cs + a * sn], 1).reshape(-1)
        assert np.array_equal(rot[i].cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert np.array_equal(rot[2].cpu().numpy().view(np.uint32), plain[2].cpu().numpy().view(np.uint32))


def test_cint8_validation(qc, synth, dev):
    import torch
    codes, scales, _ = _tensor(synth, 9, 64, 128, 1, False)
    C, S = _dev(qc, dev, codes), _dev(qc, dev, scales)
    w = qc.cint8_weights(C, S, None, 64, 128, 1)
    x = torch.zeros(128, dtype=torch.float32, device=dev)
    y = torch.full((64,), 3.0, dtype=torch.float32, device=dev)
    call = qc.cint8_project_raw
    assert call(5, [w], x, 0, 1, [y], [0]) == 3                     # mode
    assert call(0, [w], x, 0, 1, [y], [0], activation=7) == 3       # activation
    assert call(0, [w], x, 0, 0, [y], [0]) == 1                     # m
    assert call(1, [w], x, 0, 1, [y], [0]) == 1                     # SwiGLU needs two
    assert call(2, [w], x, 0, 2, [y], [0], rope_cos=x, rope_sin=x, head_dim=16) == 1
    assert call(2, [w], x, 0, 1, [y], [0], rope_cos=x, rope_sin=x, head_dim=15) == 1
    assert call(0, [qc.cint8_weights(C, S, None, 64, 128, 3)], x, 0, 1, [y], [0]) == 1
    assert call(0, [w], x, 3, 1, [y], [0]) == 2                     # storage type
    assert call(0, [w], x, 0, 1, [y], [9]) == 2
    assert call(0, [w], None, 0, 1, [y], [0]) == 3                  # nulls
    assert call(0, [w], x, 0, 1, [None], [0]) == 3
    assert call(0, [qc.cint8_weights(C, None, None, 64, 128, 1)], x, 0, 1, [y], [0]) == 3
    torch.cuda.synchronize()
    assert np.all(y.cpu().numpy() == 3.0)


@pytest.mark.parametrize("groups", [1, 32])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("fractional", [False, True])
def test_cint8_affine_codes_at_zero_point(qc, oracle, synth, dev, groups, m, fractional):
    """kInt8Affine rows (and groups) whose codes all equal the zero point
    decode to exact zeros in the reference (scale * (code - zero),
    kernels/quantization/qgemm_canonical.cpp:168-174), so such an output
    row is exactly 0 -- the contract bound is 0 there -- and a zeroed group
    adds nothing.  Integral zero points take the digit kernels' exact
    integer form; fractional ones (no code can equal them) the f32 form,
    checked against the same contract."""
    import torch
    rows, cols = 160, 4096
    codes, scales, zeros = _tensor(synth, 313 + groups, rows, cols, groups, True)
    if fractional:
        zeros = (zeros + np.float32(0.375)).astype(np.float32)
    z = zeros.reshape(rows, groups)
    g = cols // groups
    if not fractional:
        for r in (3, 64, 159):                    # whole rows at their zero points
            codes[r] = np.repeat(z[r], g).astype(np.int8)
        if groups > 1:                            # one group of row 9
            codes[9, 7 * g:8 * g] = np.int8(z[9, 7])
    keep = [_dev(qc, dev, a) for a in (codes, scales, zeros)]
    w = qc.cint8_weights(keep[0], keep[1], keep[2], rows, cols, groups)
    x = synth.normal_fast(17 + m + groups, m * cols).reshape(m, cols)
    print(f"cint8 affine at zero point groups={groups} m={m} fractional={fractional}", flush=True)
    Y = torch.full((m, rows), float("nan"), dtype=torch.float32, device=dev)
    assert qc.cint8_project_raw(0, [w], torch.from_numpy(x).to(dev), 0, m, [Y], [0]) == 0
    yf = Y.cpu().numpy()
    what = oracle.cint8_dequant(codes, scales, zeros, rows, cols, groups)
    y64, wn = oracle.cint8_project_f64(x, what)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    assert np.all(np.abs(yf - y64) <= TOL * xn * wn[None, :])
    if not fractional:
        for r in (3, 64, 159):
            assert np.all(yf[:, r] == 0.0), r


def _planes_case(qc, oracle, synth, dev, rows, cols, m, affine, seed, fractional=False):
    codes, scales, zeros = _tensor(synth, seed, rows, cols, 1, affine)
    if fractional:
        zeros = (zeros + np.float32(0.25)).astype(np.float32)
    keep = [_dev(qc, dev, a) for a in (codes, scales, zeros)]
    w = qc.cint8_weights(keep[0], keep[1], keep[2], rows, cols, 1)
    what = oracle.cint8_dequant(codes, scales, zeros, rows, cols, 1)
    return w, keep, what


def _check_contract(y, x, what):
    y64, wn = oracle_f64(x, what)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    bound = TOL * xn * wn[None, :]
    err = np.abs(y.astype(np.float64) - y64)
    assert np.all(err <= bound), float(np.max(err / np.maximum(bound, 1e-300))) * TOL


def oracle_f64(x, what):
    w = what.astype(np.float64)
    return np.asarray(x, np.float64) @ w.T, np.linalg.norm(w, axis=1)


@pytest.mark.parametrize("rows,cols,m,affine,fractional", [
    (14336, 4096, 16, False, False),      # decoder shape, symmetric channel scales
    (14336, 4096, 16, True, False),       # affine, integral zero points (exact int64 form)
    (4096, 4096, 64, True, True),         # fractional zero points (f32 form)
    (4096, 14336, 8, False, False),       # long K (down projection)
    (300, 16384, 5, True, False),         # the largest K of the route
    (1000, 2048, 512, False, False),      # prefill
    (130, 512, 1100, True, False),        # two passes of 1024 activation rows
    (70, 96, 3, False, False),            # K = 96: not a multiple of 64
])
def test_cint8_row_plane_route_contract(qc, oracle, synth, dev, rows, cols, m, affine,
                                        fractional):
    """The row-plane route (activation digit planes on the int8 MFMA GEMM,
    an exact int64 combination): every output of sampled activation rows
    within the 1e-4 normalised contract of the f64 product over the exactly
    decoded weights, and the same call on the digit-dot / f32 kernels within
    the same bound of it."""
    import torch
    print(f"cint8 planes rows={rows} cols={cols} m={m} affine={affine} frac={fractional}",
          flush=True)
    w, keep, what = _planes_case(qc, oracle, synth, dev, rows, cols, m, affine, 31 + m, fractional)
    x = synth.normal_fast(900 + m, m * cols).reshape(m, cols)
    x[0] *= np.float32(1e-30)                 # a tiny row and a huge one: per-row exponents
    if m > 2:
        x[2] *= np.float32(1e25)
    X = torch.from_numpy(x).to(dev)
    Y = torch.full((m, rows), 7.0, device=dev)
    assert qc.cint8_project_raw(0, [w], X, 0, m, [Y], [0]) == 0
    Y = Y.cpu().numpy()
    sample = sorted({0, 1, m // 2, m - 1, min(2, m - 1)})
    _check_contract(Y[sample], x[sample], what)
    qc.set_cint8_dot(1)
    try:
        Z = torch.full((m, rows), 7.0, device=dev)
        assert qc.cint8_project_raw(0, [w], X, 0, m, [Z], [0]) == 0
    finally:
        qc.set_cint8_dot(0)
    _check_contract(Z.cpu().numpy()[sample], x[sample], what)


def test_cint8_row_plane_route_epilogues(qc, oracle, synth, dev):
    """The row-plane route's epilogues at M = 6: three matrices with their
    own output types, bias + GELU on one matrix, SwiGLU over gate / up, and
    f16 / bf16 activations; each against the f32 outputs of the digit-dot
    kernels' plain projection within the contract (fused forms: against the
    f64 epilogue of those projections within a few f32 ulp)."""
    import torch
    m, cols = 6, 4096
    mats = [_planes_case(qc, oracle, synth, dev, r, cols, m, a, 70 + i)
            for i, (r, a) in enumerate(((512, False), (256, False), (256, False)))]
    x = synth.normal_fast(77, m * cols).reshape(m, cols)
    X = torch.from_numpy(x).to(dev)
    print("cint8 planes epilogues m=6", flush=True)
    ys = [torch.empty((m, r), dtype=torch.int16 if t else torch.float32, device=dev)
          for r, t in ((512, 0), (256, 1), (256, 2))]
    assert qc.cint8_project_raw(0, [w for w, _, _ in mats], X, 0, m, ys, [0, 1, 2]) == 0
    for (w, _, what), yv, t in zip(mats, ys, (0, 1, 2)):
        plain = torch.empty((m, what.shape[0]), device=dev)
        assert qc.cint8_project_raw(0, [w], X, 0, m, [plain], [0]) == 0
        p = plain.cpu().numpy()
        _check_contract(p, x, what)
        got = yv.cpu().numpy()
        if t == 1:
            assert np.array_equal(got.view(np.uint16), p.astype(np.float16).view(np.uint16))
        elif t == 2:
            assert np.array_equal(got.view(np.uint16), _bf16_bits(p))
        else:
            assert np.array_equal(got.view(np.uint32), p.view(np.uint32))
    # bias + GELU-tanh on one matrix
    w, _, what = mats[0]
    bias = torch.from_numpy(synth.normal_fast(5, 512)).to(dev)
    yb = torch.empty((m, 512), device=dev)
    assert qc.cint8_project_raw(0, [w], X, 0, m, [yb], [0], bias=bias, activation=2) == 0
    plain = torch.empty((m, 512), device=dev)
    assert qc.cint8_project_raw(0, [w], X, 0, m, [plain], [0]) == 0
    v = plain.cpu().numpy().astype(np.float64) + bias.cpu().numpy()[None, :]
    want = oracle.linear_activation_f64(v, 2)
    assert np.allclose(yb.cpu().numpy(), want, rtol=1e-5, atol=1e-6)
    # SwiGLU over two matrices of the same shape
    g, gk, gwhat = _planes_case(qc, oracle, synth, dev, 256, cols, m, True, 91)
    u, uk, uwhat = _planes_case(qc, oracle, synth, dev, 256, cols, m, True, 92)
    out = torch.empty((m, 256), device=dev)
    assert qc.cint8_project_raw(1, [g, u], X, 0, m, [out], [0]) == 0
    pg, pu = torch.empty((m, 256), device=dev), torch.empty((m, 256), device=dev)
    assert qc.cint8_project_raw(0, [g, u], X, 0, m, [pg, pu], [0, 0]) == 0
    gv = pg.cpu().numpy().astype(np.float64)
    want = gv / (1.0 + np.exp(-gv)) * pu.cpu().numpy().astype(np.float64)
    assert np.allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6)
    # 16-bit activations decode exactly: the f32 call on the decoded values
    for t in (1, 2):
        if t == 1:
            xh = x.astype(np.float16)
            Xt = torch.from_numpy(xh.view(np.int16).copy()).to(dev)
            xd = xh.astype(np.float32)
        else:
            xb = _bf16_bits(x)
            Xt = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
            xd = (xb.astype(np.uint32) << 16).view(np.float32).reshape(m, cols)
        a = torch.empty((m, 512), device=dev)
        b = torch.empty((m, 512), device=dev)
        assert qc.cint8_project_raw(0, [mats[0][0]], Xt, t, m, [a], [0]) == 0
        assert qc.cint8_project_raw(0, [mats[0][0]], torch.from_numpy(xd).to(dev), 0, m, [b],
                                    [0]) == 0
        assert np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("m,rows", [(2, 300), (12, 300), (20, 96), (40, 1000), (64, 130),
                                    (100, 200)])
def test_cint8_row_plane_swiglu_sizes(qc, oracle, synth, dev, m, rows):
    """SwiGLU on the row-plane route (gate and up paired in one GEMM) at each
    tile size of the one-launch form, above 64 rows (the finish kernel), and
    at row counts that are not a multiple of 32: every finite output within
    a few f32 ulp of SiLU(gate) * up over the same call's plain projections
    (themselves within the contract of the f64 oracle), and the row holding
    +inf in the class those projections give."""
    import torch
    cols = 1024
    affine = m % 4 == 0                   # both matrices alike (a call's matrices share the form)
    g, gk, gwhat = _planes_case(qc, oracle, synth, dev, rows, cols, m, affine, 101 + m)
    u, uk, uwhat = _planes_case(qc, oracle, synth, dev, rows, cols, m, affine, 202 + m)
    x = synth.normal_fast(303 + m, m * cols).reshape(m, cols)
    bad = m - 1
    x[bad, 5] = np.inf
    X = torch.from_numpy(x).to(dev)
    print(f"cint8 planes swiglu m={m} rows={rows}", flush=True)
    out = torch.full((m, rows), 7.0, device=dev)
    assert qc.cint8_project_raw(1, [g, u], X, 0, m, [out], [0]) == 0
    pg, pu = torch.empty((m, rows), device=dev), torch.empty((m, rows), device=dev)
    assert qc.cint8_project_raw(0, [g, u], X, 0, m, [pg, pu], [0, 0]) == 0
    pg, pu, out = pg.cpu().numpy(), pu.cpu().numpy(), out.cpu().numpy()
    fin = [r for r in range(m) if r != bad]
    _check_contract(pg[fin], x[fin], gwhat)
    _check_contract(pu[fin], x[fin], uwhat)
    gv = pg.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        want = gv / (1.0 + np.exp(-gv)) * pu.astype(np.float64)
    assert np.allclose(out[fin], want[fin], rtol=1e-5, atol=1e-6)
    for got, ref in ((np.isnan(out[bad]), np.isnan(want[bad])),
                     (np.isposinf(out[bad]), np.isposinf(want[bad])),
                     (np.isneginf(out[bad]), np.isneginf(want[bad]))):
        assert np.array_equal(got, ref), np.flatnonzero(got != ref)[:5]


@pytest.mark.parametrize("groups,affine,fractional,m,mode,wide", [
    (16, False, False, 12, 0, False),   # groups of 128 columns
    (16, True, False, 3, 0, False),     # integral zero points (exact int32 group sums), 3 rows
    (8, True, True, 40, 0, False),      # groups of 256, fractional zero points (f32 form)
    (4, True, False, 100, 0, False),    # groups of 512 above 64 rows (256 x 128 tiles)
    (4, True, False, 24, 0, True),      # integral zero points past the int32 bound (int64)
    (16, True, False, 20, 1, False),    # SwiGLU with group scales
    (32, False, False, 12, 0, False),   # groups of 64 columns (half-line K steps)
    (32, True, False, 40, 0, False),
    (32, True, True, 100, 0, False),
    (32, True, False, 6, 1, False),
    (64, False, False, 12, 0, False),   # groups of 32 columns (two folds per K step)
    (64, True, False, 40, 0, False),
    (64, True, True, 100, 0, False),
    (64, True, False, 8, 1, False),
    (64, True, False, 24, 0, False),    # 8-wave 128 x 64 tiles, B loads on waves 0..3
    (32, True, True, 28, 1, False),     # SwiGLU, groups of 64, 8-wave 128 x 128 tiles
])
def test_cint8_row_plane_route_groups(qc, oracle, synth, dev, groups, affine, fractional, m,
                                      mode, wide):
    """Group-scaled weights on the row-plane route (groups of 64 or a multiple
    of 128 columns): each group's plane sums folded into f32 at the end of its
    last K step.  Every finite output within the 1e-4 normalised contract of the f64
    product over the exactly decoded weights (SwiGLU: within a few f32 ulp of
    the f64 epilogue of the same call's plain projections), an activation row
    holding +-inf in the class of the digit-dot kernels' result, and a weight
    row whose codes all equal their integral zero points exactly 0.  `wide`:
    rows 20-29 get integral zero points near 4e4, past the bound (32639 for
    groups of 512) up to which D_t - z S_t is formed in int32."""
    import torch
    rows, cols = 300, 2048
    print(f"cint8 planes groups={groups} affine={affine} frac={fractional} m={m} mode={mode} "
          f"wide={wide}", flush=True)
    mats = []
    for i in range(2 if mode == 1 else 1):
        codes, scales, zeros = _tensor(synth, 500 + 7 * i + groups, rows, cols, groups, affine)
        if affine and fractional:
            zeros = (zeros + np.float32(0.25)).astype(np.float32)
        if wide:
            zeros[20 * groups:30 * groups] += np.float32(40000)
        if affine and not fractional:
            g = cols // groups
            codes[7] = np.repeat(zeros[7 * groups:8 * groups], g).astype(np.int8)   # w_hat row 7 = 0
        keep = [_dev(qc, dev, a) for a in (codes, scales, zeros)]
        w = qc.cint8_weights(keep[0], keep[1], keep[2], rows, cols, groups)
        what = oracle.cint8_dequant(codes, scales, zeros, rows, cols, groups)
        mats.append((w, keep, what))
    x = synth.normal_fast(600 + m, m * cols).reshape(m, cols)
    x[0] *= np.float32(1e-20)
    bad = m - 1
    x[bad, 33] = -np.inf
    X = torch.from_numpy(x).to(dev)
    fin = [r for r in range(m) if r != bad]
    ws = [w for w, _, _ in mats]
    Y = torch.full((m, rows), 7.0, device=dev)
    assert qc.cint8_project_raw(mode, ws, X, 0, m, [Y], [0]) == 0
    Y = Y.cpu().numpy()
    qc.set_cint8_dot(1)
    try:
        Z = torch.full((m, rows), 7.0, device=dev)
        assert qc.cint8_project_raw(mode, ws, X, 0, m, [Z], [0]) == 0
    finally:
        qc.set_cint8_dot(0)
    Z = Z.cpu().numpy()
    for got, ref in ((np.isnan(Y[bad]), np.isnan(Z[bad])),
                     (np.isposinf(Y[bad]), np.isposinf(Z[bad])),
                     (np.isneginf(Y[bad]), np.isneginf(Z[bad]))):
        assert np.array_equal(got, ref), np.flatnonzero(got != ref)[:5]
    if mode == 0:
        _check_contract(Y[fin], x[fin], mats[0][2])
        if affine and not fractional:
            assert np.all(Y[fin, 7] == 0.0)
    else:
        pg, pu = torch.empty((m, rows), device=dev), torch.empty((m, rows), device=dev)
        assert qc.cint8_project_raw(0, ws, X, 0, m, [pg, pu], [0, 0]) == 0
        pg, pu = pg.cpu().numpy(), pu.cpu().numpy()
        _check_contract(pg[fin], x[fin], mats[0][2])
        _check_contract(pu[fin], x[fin], mats[1][2])
        gv = pg.astype(np.float64)
        with np.errstate(invalid="ignore", over="ignore"):   # the +-inf row
            want = gv / (1.0 + np.exp(-gv)) * pu.astype(np.float64)
        assert np.allclose(Y[fin], want[fin], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rows,cols,groups,m", [
    (200, 16384, 512, 6),     # the largest K: 512 groups of 32
    (200, 16384, 256, 6),     # 256 groups of 64
    (200, 16384, 128, 40),    # 128 groups of 128
    (130, 512, 16, 1100),     # groups of 32 over two chunks of activation rows
])
def test_cint8_row_plane_route_groups_sizes(qc, oracle, synth, dev, rows, cols, groups, m):
    """Group-scaled weights on the row-plane route at the largest K (the most
    groups the prep's per-group digit sums hold) and with more activation rows
    than one pass takes: every output within the 1e-4 normalised contract of
    the f64 product over the exactly decoded weights (affine, integral zero
    points)."""
    import torch
    print(f"cint8 planes groups sizes rows={rows} cols={cols} groups={groups} m={m}", flush=True)
    codes, scales, zeros = _tensor(synth, 900 + groups, rows, cols, groups, True)
    keep = [_dev(qc, dev, a) for a in (codes, scales, zeros)]
    w = qc.cint8_weights(keep[0], keep[1], keep[2], rows, cols, groups)
    what = oracle.cint8_dequant(codes, scales, zeros, rows, cols, groups)
    x = synth.normal_fast(950 + m, m * cols).reshape(m, cols)
    X = torch.from_numpy(x).to(dev)
    Y = torch.full((m, rows), 7.0, device=dev)
    assert qc.cint8_project_raw(0, [w], X, 0, m, [Y], [0]) == 0
    _check_contract(Y.cpu().numpy(), x, what)


def test_cint8_row_plane_route_nonfinite_rows(qc, oracle, synth, dev):
    """Activation rows holding +-inf or NaN on the row-plane route: those
    rows get the reference's f32 result class per output, the finite rows
    are bit-identical to the same call with the bad rows zeroed."""
    import torch
    rows, cols, m = 300, 4096, 6
    codes, scales, zeros = _tensor(synth, 55, rows, cols, 1, True)
    codes[:, 200] = 0
    zeros[::5] = 0.0
    keep = [_dev(qc, dev, a) for a in (codes, scales, zeros)]
    w = qc.cint8_weights(keep[0], keep[1], keep[2], rows, cols, 1)
    what = oracle.cint8_dequant(codes, scales, zeros, rows, cols, 1).astype(np.float64)
    x = synth.normal_fast(66, m * cols).reshape(m, cols)
    x[1, 200] = np.inf
    x[3, 77] = -np.inf
    x[3, 3000] = np.inf
    x[4, 1234] = np.nan
    print("cint8 planes nonfinite rows", flush=True)
    Y = torch.empty((m, rows), device=dev)
    assert qc.cint8_project_raw(0, [w], torch.from_numpy(x).to(dev), 0, m, [Y], [0]) == 0
    Y = Y.cpu().numpy()
    xz = x.copy()
    xz[[1, 3, 4]] = 0.0
    Z = torch.empty((m, rows), device=dev)
    assert qc.cint8_project_raw(0, [w], torch.from_numpy(xz).to(dev), 0, m, [Z], [0]) == 0
    Z = Z.cpu().numpy()
    for r in (0, 2, 5):
        assert np.array_equal(Y[r].view(np.uint32), Z[r].view(np.uint32)), r
    for r in (1, 3, 4):
        with np.errstate(invalid="ignore", over="ignore"):
            y64 = (what * x[r].astype(np.float64)[None, :]).sum(axis=1)
        for got, want in ((np.isnan(Y[r]), np.isnan(y64)), (np.isposinf(Y[r]), np.isposinf(y64)),
                          (np.isneginf(Y[r]), np.isneginf(y64))):
            assert np.array_equal(got, want), (r, np.flatnonzero(got != want)[:5])
