"""Calls captured into a HIP graph (torch.cuda.graph) and replayed.

Each case runs the call eagerly on a stream (which also sizes that stream's
scratch cache), captures the same call on that stream, then replays the graph
three times on it with eager work queued between the replays (the outputs
refilled, and the same entry point run on other inputs, sharing the stream's
scratch in stream order).  Every replay must reproduce the eager outputs bit
for bit: the captured launches hold no memset node and no per-call
allocation, and the scratch a graph keeps is the stream's own.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _fill(t):
    if t.dtype.is_floating_point:
        t.fill_(float("nan"))
    else:
        t.fill_(85)


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint8).copy()


def _ok(status):
    assert status == 0, status


def _replay(call, outs, other):
    """call(): the captured work; other(): an eager call of the same entry
    point on other inputs and outputs."""
    import torch
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        call()
    torch.cuda.synchronize()
    want = [_bits(o) for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call()
    torch.cuda.synchronize()
    for rep in range(3):
        with torch.cuda.stream(s):
            for o in outs:
                _fill(o)
            other()
            g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert np.array_equal(_bits(o), w), rep
    del g


def _packed(qc, dev, fmt, n, k, seed):
    import torch
    gen = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn((n, k), generator=gen, device=dev)
    return qc.pack(fmt, w)


@pytest.mark.parametrize("fmt,m,n", [(1, 1, 2048), (0, 4, 4096), (1, 8, 4096), (0, 16, 4096),
                                     (0, 32, 14336), (1, 128, 1024)])
def test_qgemv_qgemm_graph_replay(qc, dev, fmt, m, n):
    """qgemv (m = 1) and qgemm at m = 4 (rows route), 8 (digit MFMA, digits
    built in the GEMM, K split four ways + reduce), 16 / 32 (prep + f16 MFMA,
    K split) and 128 (the 2-D route)."""
    import torch
    k = 4096
    print(f"graph qgemm fmt={fmt} m={m} n={n}", flush=True)
    P = _packed(qc, dev, fmt, n, k, 5 + m)
    gen = torch.Generator(device=dev).manual_seed(7 + m)
    x = torch.randn((m, k), generator=gen, device=dev)
    x2 = torch.randn((m, k), generator=gen, device=dev)
    y = torch.empty((m, n), device=dev)
    y2 = torch.empty((m, n), device=dev)
    if m == 1:
        call = lambda: qc.qgemv_raw(fmt, P, x, y, n, k)
        other = lambda: qc.qgemv_raw(fmt, P, x2, y2, n, k)
    else:
        call = lambda: qc.qgemm_raw(fmt, P, x, y, m, n, k)
        other = lambda: qc.qgemm_raw(fmt, P, x2, y2, m, n, k)
    _replay(lambda: _ok(call()), [y], lambda: _ok(other()))


@pytest.mark.parametrize("mode,m,rows,groups", [(0, 16, 4096, 1), (0, 3, 1000, 1),
                                                (1, 16, 2048, 1), (1, 100, 512, 1),
                                                (0, 300, 1024, 1), (0, 24, 2048, 16),
                                                (1, 8, 1024, 16), (0, 40, 1024, 32),
                                                (1, 12, 1024, 64)])
def test_cint8_project_graph_replay(qc, dev, mode, m, rows, groups):
    """Canonical int8 projections on the row-plane route (plain and SwiGLU,
    row scales and groups of 128 or 64 columns), each call a prep and one GEMM
    per matrix with the scratch from the stream's cache."""
    import torch
    k = 2048
    print(f"graph cint8 mode={mode} m={m} rows={rows} groups={groups}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(11 + m)
    keep, ws = [], []
    for _ in range(2 if mode == 1 else 1):
        codes = torch.randint(-127, 128, (rows, k), generator=gen, device=dev, dtype=torch.int8)
        scales = torch.rand(rows * groups, generator=gen, device=dev) * 1e-3 + 1e-5
        zeros = torch.randint(-4, 5, (rows * groups,), generator=gen, device=dev).float()
        keep += [codes, scales, zeros]
        ws.append(qc.cint8_weights(codes, scales, zeros, rows, k, groups))
    x = torch.randn((m, k), generator=gen, device=dev)
    x2 = torch.randn((m, k), generator=gen, device=dev)
    y = torch.empty((m, rows), device=dev)
    y2 = torch.empty((m, rows), device=dev)
    call = lambda: _ok(qc.cint8_project_raw(mode, ws, x, 0, m, [y], [0]))
    other = lambda: _ok(qc.cint8_project_raw(mode, ws, x2, 0, m, [y2], [0]))
    _replay(call, [y], other)


def test_w8a8_graph_replay(qc, dev):
    """quantize_int8 and the W8A8 GEMM with a device status (cleared by a fill
    kernel inside the graph; a NULL status would make the calls synchronous,
    which capture does not allow), and the affine canonical W8A8 route (weight
    row sums in the stream's scratch)."""
    import torch
    m, n, k = 256, 1024, 1024
    print("graph w8a8", flush=True)
    gen = torch.Generator(device=dev).manual_seed(23)
    x = torch.randn((m, k), generator=gen, device=dev)
    x2 = torch.randn((m, k), generator=gen, device=dev)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8)
    ws = torch.rand(n, generator=gen, device=dev) * 1e-2
    codes = torch.empty((m, k), dtype=torch.int8, device=dev)
    scales = torch.empty((m, 1), device=dev)
    codes2 = torch.empty_like(codes)
    scales2 = torch.empty_like(scales)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    status2 = torch.zeros(1, dtype=torch.int32, device=dev)
    y = torch.empty((m, n), device=dev)
    y2 = torch.empty((m, n), device=dev)

    def call():
        status.zero_()
        _ok(qc.quantize_int8_raw(x, codes, scales, m, k, 0, status))
        _ok(qc.int8_gemm_raw(w, codes, ws, scales, None, None, y, m, n, k, dev_status=status))

    def other():
        status2.zero_()
        _ok(qc.quantize_int8_raw(x2, codes2, scales2, m, k, 0, status2))
        _ok(qc.int8_gemm_raw(w, codes2, ws, scales2, None, None, y2, m, n, k,
                             dev_status=status2))

    _replay(call, [codes, scales, y, status], other)

    # canonical W8A8 with affine activations: integer zero points
    wt = qc.cint8_weights(w, ws, None, n, k, 1)
    a_codes = torch.randint(-128, 128, (m, k), generator=gen, device=dev, dtype=torch.int8)
    a_scales = torch.rand(m, generator=gen, device=dev) * 1e-2
    a_zeros = torch.randint(-20, 21, (m,), generator=gen, device=dev)
    a_zf = a_zeros.float()
    at = qc.cint8_weights(a_codes, a_scales, a_zf, m, k, 1)
    zi = a_zeros.to(torch.int32)
    z = torch.empty((m, n), device=dev)
    z2 = torch.empty((m, n), device=dev)
    _replay(lambda: _ok(qc.cint8_quantized_gemm_raw(wt, at, z, zi)), [z],
            lambda: _ok(qc.cint8_quantized_gemm_raw(wt, at, z2, zi)))
