"""GPU parity: quantize_int8 codes/scales and q8_0/q4_0 pack/unpack, bit-exact
against the oracle (which is pinned bit-exactly to the reference's own
functions in tests/test_oracle.py)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _quant_check(qc, oracle, dev, x, group=0):
    import torch
    st, c_want, s_want = oracle.quantize_int8(x, group)
    assert st == 0
    c, s = qc.quantize_int8(torch.from_numpy(x).to(dev), group)
    assert np.array_equal(c.cpu().numpy(), c_want)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_want.view(np.uint32))


def test_quantize_int8_config3(qc, oracle, synth, dev):
    """BASELINE config 3 activations: 2048 x 4096 with 0.1% outliers x20."""
    print("quantize_int8 2048x4096", flush=True)
    x = synth.activations_outliers_fast(3, 2048, 4096)
    _quant_check(qc, oracle, dev, x)


@pytest.mark.parametrize("rows,dim,group", [(1, 4, 0), (3, 100, 0), (5, 1024, 0), (7, 2048, 0),
                                            (3, 8192, 0), (2, 12288, 0), (4, 4096, 128),
                                            (2, 4, 2), (3, 96, 32), (5, 14336, 0), (2, 16384, 0),
                                            (3, 16388, 0), (2, 32768, 0), (2, 32772, 0),
                                            (3, 14338, 0)])
def test_quantize_int8_shapes(qc, oracle, dev, rows, dim, group):
    rng = np.random.default_rng(rows * 1000 + dim)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    x[0, : min(dim, 8)] = 0.0
    _quant_check(qc, oracle, dev, x, group)


def test_quantize_int8_down_proj(qc, oracle, synth, dev):
    """Config 4's down projection input: 512 x 14336 with outliers (a 512-thread
    workgroup per row)."""
    print("quantize_int8 512x14336", flush=True)
    x = synth.activations_outliers_fast(4, 512, 14336)
    _quant_check(qc, oracle, dev, x)


def test_quantize_int8_edges(qc, oracle, dev):
    x = np.zeros((3, 256), np.float32)                       # all-zero rows
    x[1] = (np.arange(256, dtype=np.float32) - 128) * np.float32(0.5)   # ties
    x[2] = np.float32(1e-38) * np.arange(256, dtype=np.float32)          # subnormals
    _quant_check(qc, oracle, dev, x)
    # known answer (tests/correctness/test_quantization.cpp:100-111)
    x = np.array([[-2.0, -0.5, 0.0, 2.0], [1.0, 2.0, 3.0, 4.0]], np.float32)
    _quant_check(qc, oracle, dev, x, 2)


def test_quantize_int8_nonfinite(qc, dev):
    import torch
    x = torch.ones((4, 1024), dtype=torch.float32, device=dev)
    x[2, 5] = float("nan")
    codes = torch.full((4, 1024), 7, dtype=torch.int8, device=dev)
    scales = torch.full((4, 1), 9.0, dtype=torch.float32, device=dev)
    # synchronous reference semantics: status 3, outputs untouched
    assert qc.quantize_int8_raw(x, codes, scales, 4, 1024) == 3
    assert torch.all(codes == 7) and torch.all(scales == 9.0)
    # asynchronous form: finite rows written, the bad row untouched, status word 3
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    assert qc.quantize_int8_raw(x, codes, scales, 4, 1024, 0, status) == 0
    torch.cuda.synchronize()
    assert int(status.item()) == 3
    assert torch.all(codes[2] == 7) and float(scales[2, 0]) == 9.0
    assert torch.all(codes[0] == 127)
    # validation order (kernels/quantization/quantization_ref.cpp:143-147)
    assert qc.quantize_int8_raw(x, codes, scales, 4, 1024, 3) == 1
    assert qc.quantize_int8_raw(None, codes, scales, 4, 1024) == 3


@pytest.mark.parametrize("fmt", [0, 1])
def test_pack_unpack_bit_exact(qc, oracle, synth, dev, fmt):
    import torch
    print(f"pack fmt={fmt}", flush=True)
    n, k = 1024, 4096
    w = synth.weights(0, n, k)
    edge = np.zeros((8, k), np.float32)
    edge[0] = 1e-3
    edge[1] = np.linspace(-1, 1, k)
    edge[2] = (np.arange(k, dtype=np.float32) % 32 - 16) * np.float32(0.5)
    edge[3, ::32] = 3.0e38
    w = np.concatenate([w, edge])
    n = w.shape[0]
    st, want = oracle.pack(fmt, w)
    got = qc.pack(fmt, torch.from_numpy(w).to(dev)).cpu().numpy()
    assert np.array_equal(got, want)
    un = qc.unpack(fmt, torch.from_numpy(want).to(dev), n, k).cpu().numpy()
    assert np.array_equal(un.view(np.uint32), oracle.unpack(fmt, want, n, k).view(np.uint32))


def test_pack_rejects_nonfinite(qc, dev):
    import torch
    w = torch.ones((2, 64), dtype=torch.float32, device=dev)
    w[1, 40] = float("inf")
    out = torch.zeros(2 * 2 * 34, dtype=torch.uint8, device=dev)
    assert qc.pack_raw(0, w, out, 2, 64) == 3


def test_sync_status_concurrent_streams(qc, dev):
    """Synchronous calls (dev_status NULL) from two host threads on two streams:
    each call has its own device flag, so a non-finite input on one stream
    never leaks its status 3 into the other stream's finite calls (or is lost)."""
    import threading
    import torch
    rows, dim = 64, 256
    x_bad = torch.ones(rows, dim, device=dev)
    x_bad[5, 7] = float("nan")
    x_ok = torch.ones(rows, dim, device=dev)
    streams = {"bad": torch.cuda.Stream(), "ok": torch.cuda.Stream()}
    results = {"bad": [], "ok": []}

    def run(name, x):
        codes = torch.empty(rows, dim, dtype=torch.int8, device=dev)
        scales = torch.empty(rows, device=dev)
        s = streams[name].cuda_stream
        for _ in range(300):
            results[name].append(qc.quantize_int8_raw(x, codes, scales, rows, dim, 0, None, s))

    print("sync status from two threads", flush=True)
    threads = [threading.Thread(target=run, args=(nm, x)) for nm, x in (("bad", x_bad), ("ok", x_ok))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    torch.cuda.synchronize()
    assert len(results["bad"]) == 300 and len(results["ok"]) == 300
    assert set(results["bad"]) == {3} and set(results["ok"]) == {0}
