"""GPU parity: fused decode projections (qgemv_up_gate, qgemv_up_gate_activation,
qgemv_qkv, qgemv_qkv_rope_kv; kernels/quantization/qgemv_fused_ref.cpp:184-443)
through the C ABI.

Each projection of the fused launch uses the GEMV's per-row arithmetic, so it
is bit-identical to qc_hip_qgemv of that matrix (itself held to the 1e-4
contract against the f64 oracle in test_gpu_gemv.py), and also checked against
the f64 oracle here.  The RoPE seam's outputs are bit-identical to the
reference's rotation (out[d] = a*c - b*s, out[d+half] = b*c + a*s, each
operation rounded in f32) applied to those projections, with every other
cache slot left as it was.  The activation form is checked against
activation(gate) * up evaluated in f64 from the plain fused projections.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _packed(oracle, synth, fmt, n, k, seed):
    w = synth.normal_fast(seed, n * k, 0.02).reshape(n, k)
    st, p = oracle.pack(fmt, w)
    assert st == 0
    return p


def _dev(arr, dev, offset=0):
    import torch
    t = torch.zeros(arr.size + offset, dtype=torch.uint8 if arr.dtype == np.uint8 else torch.float32,
                    device=dev)
    t[offset:] = torch.from_numpy(arr).to(dev)
    return t[offset:]


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _check_contract(oracle, fmt, packed, x, y, n, k):
    y64, wn = oracle.gemv_f64(fmt, packed, x, n, k)
    ok, worst = oracle.within_contract(y, y64, wn, x, TOL)
    assert ok, worst


# w_off: weights 2 bytes off 4-byte alignment; x_off: x one or three floats
# off 16-byte alignment (both take the per-matrix route)
@pytest.mark.parametrize("fmt,n,k,w_off,x_off", [(1, 14336, 4096, 0, 0), (0, 4096, 4096, 0, 0),
                                                 (1, 300, 64, 0, 0), (0, 1000, 96, 0, 0),
                                                 (1, 257, 4096, 2, 0), (0, 70, 14336, 0, 0),
                                                 (1, 1024, 4096, 0, 1), (0, 300, 96, 0, 3)])
def test_up_gate(qc, oracle, synth, dev, fmt, n, k, w_off, x_off):
    import torch
    print(f"up_gate fmt={fmt} n={n} k={k} w_off={w_off} x_off={x_off}", flush=True)
    pu = _packed(oracle, synth, fmt, n, k, 10 + n)
    pg = _packed(oracle, synth, fmt, n, k, 20 + n)
    x = synth.normal_fast(30 + k, k)
    PU, PG, X = _dev(pu, dev, w_off), _dev(pg, dev, w_off), _dev(x, dev, x_off)
    up = torch.empty(n, dtype=torch.float32, device=dev)
    gate = torch.empty(n, dtype=torch.float32, device=dev)
    assert qc.qgemv_up_gate_raw(fmt, PU, PG, X, up, gate, n, k) == 0
    up, gate = up.cpu().numpy(), gate.cpu().numpy()
    assert np.array_equal(_bits(up), _bits(qc.qgemv(fmt, PU, X, n, k).cpu().numpy()))
    assert np.array_equal(_bits(gate), _bits(qc.qgemv(fmt, PG, X, n, k).cpu().numpy()))
    for p, y in ((pu, up), (pg, gate)):
        _check_contract(oracle, fmt, p, x, y, n, k)


def _act64(v, gelu):
    v = v.astype(np.float64)
    if gelu:
        return 0.5 * v * (1.0 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))
    return v / (1.0 + np.exp(-v))


@pytest.mark.parametrize("fmt,n,k,x_off", [(1, 14336, 4096, 0), (0, 512, 4096, 0),
                                           (1, 130, 96, 0), (0, 700, 4096, 1), (1, 96, 160, 2)])
@pytest.mark.parametrize("gelu", [True, False])
def test_up_gate_activation(qc, oracle, synth, dev, fmt, n, k, x_off, gelu):
    import torch
    print(f"up_gate_activation fmt={fmt} n={n} k={k} x_off={x_off} gelu={gelu}", flush=True)
    pu = _packed(oracle, synth, fmt, n, k, 40 + n)
    pg = _packed(oracle, synth, fmt, n, k, 50 + n)
    x = synth.normal_fast(60 + k, k) * np.float32(3.0)     # gate values over several units
    PU, PG, X = _dev(pu, dev), _dev(pg, dev), _dev(x, dev, x_off)
    up = torch.empty(n, dtype=torch.float32, device=dev)
    gate = torch.empty(n, dtype=torch.float32, device=dev)
    out = torch.empty(n, dtype=torch.float32, device=dev)
    assert qc.qgemv_up_gate_raw(fmt, PU, PG, X, up, gate, n, k) == 0
    assert qc.qgemv_up_gate_activation_raw(fmt, PU, PG, X, out, n, k, gelu) == 0
    up, gate, out = (t.cpu().numpy() for t in (up, gate, out))
    want = _act64(gate, gelu) * up.astype(np.float64)
    # f32 activation rounding (a few ulp) plus, for GELU-tanh, the cancellation
    # in 1 + tanh(z) for negative gates (~ulp(1) * |gate|)
    bound = 1e-5 * np.abs(gate.astype(np.float64) * up) + 2e-6 * np.abs(want) + 1e-30
    assert np.all(np.abs(out - want) <= bound)
    # and against the f64 oracle's projections
    g64, _ = oracle.gemv_f64(fmt, pg, x, n, k)
    u64, _ = oracle.gemv_f64(fmt, pu, x, n, k)
    ref = _act64(g64, gelu) * u64
    scale = np.max(np.abs(ref)) + 1e-30
    assert np.max(np.abs(out - ref)) <= 1e-3 * scale


@pytest.mark.parametrize("fmt,qd,kvd,k,x_off", [(1, 4096, 1024, 4096, 0), (0, 300, 64, 256, 0),
                                                (1, 96, 32, 160, 0), (0, 2048, 512, 8192, 0),
                                                (1, 512, 128, 4096, 1)])
def test_qkv(qc, oracle, synth, dev, fmt, qd, kvd, k, x_off):
    import torch
    print(f"qkv fmt={fmt} q={qd} kv={kvd} k={k} x_off={x_off}", flush=True)
    pq = _packed(oracle, synth, fmt, qd, k, 70)
    pk = _packed(oracle, synth, fmt, kvd, k, 71)
    pv = _packed(oracle, synth, fmt, kvd, k, 72)
    x = synth.normal_fast(73 + k, k)
    PQ, PK, PV, X = _dev(pq, dev), _dev(pk, dev), _dev(pv, dev), _dev(x, dev, x_off)
    q = torch.empty(qd, dtype=torch.float32, device=dev)
    ko = torch.empty(kvd, dtype=torch.float32, device=dev)
    vo = torch.empty(kvd, dtype=torch.float32, device=dev)
    assert qc.qgemv_qkv_raw(fmt, PQ, PK, PV, X, q, ko, vo, qd, kvd, k) == 0
    for P, p, y, n in ((PQ, pq, q, qd), (PK, pk, ko, kvd), (PV, pv, vo, kvd)):
        y = y.cpu().numpy()
        assert np.array_equal(_bits(y), _bits(qc.qgemv(fmt, P, X, n, k).cpu().numpy()))
        _check_contract(oracle, fmt, p, x, y, n, k)


def _rope_f32(y, heads, hd, c, sn):
    """The reference's rotation in f32 (qgemv_fused_ref.cpp:398-433)."""
    v = y.reshape(heads, 2, hd // 2)
    a, b = v[:, 0], v[:, 1]
    return np.stack([a * c - b * sn, b * c + a * sn], axis=1).reshape(-1).astype(np.float32)


# (fmt, query heads, kv heads, head_dim, K, slots, position, slot, x offset, w offset)
@pytest.mark.parametrize("fmt,qh,kvh,hd,k,slots,pos,slot,x_off,w_off", [
    (1, 32, 8, 128, 4096, 4, 17, 2, 0, 0),    # config 4's attention shape (one launch)
    (0, 32, 8, 128, 4096, 2, 5, 0, 0, 0),
    (1, 8, 2, 64, 4096, 3, 3, -1, 0, 0),      # slot -1: Q only
    (0, 4, 4, 6, 512, 2, 0, 1, 0, 0),         # half = 3
    (1, 2, 1, 6, 96, 3, 1, 2, 0, 0),          # odd K/32: per-matrix route
    (0, 8, 2, 64, 512, 2, 2, 1, 1, 0),        # misaligned x: per-matrix route
    (1, 4, 2, 32, 256, 2, 2, 0, 0, 2),        # misaligned W: per-matrix route
])
def test_qkv_rope_kv(qc, oracle, synth, dev, fmt, qh, kvh, hd, k, slots, pos, slot, x_off, w_off):
    import torch
    print(f"qkv_rope_kv fmt={fmt} heads={qh}/{kvh} hd={hd} k={k} slot={slot} x_off={x_off} "
          f"w_off={w_off}", flush=True)
    qd, kvd, half = qh * hd, kvh * hd, hd // 2
    pq = _packed(oracle, synth, fmt, qd, k, 80)
    pk = _packed(oracle, synth, fmt, kvd, k, 81)
    pv = _packed(oracle, synth, fmt, kvd, k, 82)
    x = synth.normal_fast(83 + k, k)
    max_pos = pos + 3
    ang = synth.normal_fast(84, max_pos * half).reshape(max_pos, half) * np.float32(3.0)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    PQ, PK, PV = _dev(pq, dev, w_off), _dev(pk, dev, w_off), _dev(pv, dev, w_off)
    X, C, S = _dev(x, dev, x_off), _dev(cos.reshape(-1), dev), _dev(sin.reshape(-1), dev)
    fill = np.arange(slots * kvd, dtype=np.float32) + np.float32(0.5)
    KC, VC = _dev(fill, dev), _dev(-fill, dev)
    q = torch.full((qd,), 7.0, dtype=torch.float32, device=dev)
    assert qc.qgemv_qkv_rope_kv_raw(fmt, PQ, PK, PV, X, C, S, q, KC, VC, qh, kvh, hd, k, slots,
                                    max_pos, pos, slot) == 0
    plain = [qc.qgemv(fmt, P, X, n, k).cpu().numpy() for P, n in ((PQ, qd), (PK, kvd), (PV, kvd))]
    for p, y, n in zip((pq, pk, pv), plain, (qd, kvd, kvd)):
        _check_contract(oracle, fmt, p, x, y, n, k)
    c, sn = cos[pos], sin[pos]
    assert np.array_equal(_bits(q.cpu().numpy()), _bits(_rope_f32(plain[0], qh, hd, c, sn)))
    kc, vc = KC.cpu().numpy(), VC.cpu().numpy()
    keep = np.ones(slots * kvd, bool)
    if slot >= 0:
        sl = slice(slot * kvd, (slot + 1) * kvd)
        keep[sl] = False
        assert np.array_equal(_bits(kc[sl]), _bits(_rope_f32(plain[1], kvh, hd, c, sn)))
        assert np.array_equal(_bits(vc[sl]), _bits(plain[2]))
    assert np.array_equal(kc[keep], fill[keep]) and np.array_equal(vc[keep], -fill[keep])


def test_qkv_rope_kv_validation(qc, oracle, synth, dev):
    import torch
    pq = _dev(_packed(oracle, synth, 0, 8, 64, 90), dev)
    x, cs = _dev(synth.normal_fast(91, 64), dev), _dev(np.ones(8, np.float32), dev)
    q = torch.zeros(8, dtype=torch.float32, device=dev)
    kc = torch.zeros(16, dtype=torch.float32, device=dev)
    call = lambda fmt=0, hd=4, pos=1, slot=0, ptr=pq, k=64, maxp=4: qc.qgemv_qkv_rope_kv_raw(
        fmt, ptr, pq, pq, x, cs, cs, q, kc, kc, 2, 1, hd, k, 2, maxp, pos, slot)
    assert call(hd=3) == 1 and call(pos=4) == 1 and call(pos=-1) == 1 and call(slot=2) == 1
    assert call(slot=-2) == 1 and call(k=48) == 1
    assert call(ptr=None) == 3
    assert call(fmt=5) == 2
    torch.cuda.synchronize()
    assert np.all(q.cpu().numpy() == 0) and np.all(kc.cpu().numpy() == 0)
    assert call() == 0
