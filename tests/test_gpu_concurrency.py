"""GPU: qgemm calls from several host threads at once on one stream.

The reference allows concurrent invocations (include/quixicore_cpu/workspace.h:
17-18).  The GPU library keeps per-stream scratch for qgemm (activation
fragments, partial sums, row exponents); the calls here share one fresh
stream, so their first calls also race to grow that scratch.  Each thread's
results must be bit-identical to the same call made alone, and within the
contract bound of the f64 oracle.
"""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_qgemm_threads_share_one_stream(qc, oracle, synth, dev):
    import torch
    fmt, n, k = 0, 2048, 4096
    print(f"qgemm threads fmt={fmt} n={n} k={k}", flush=True)
    w = synth.normal_fast(77, n * k, 0.02).reshape(n, k)
    st, packed = oracle.pack(fmt, w)
    assert st == 0
    P = torch.from_numpy(packed).to(dev)
    # digit mode (M=4), passes of dense tiles (M=40) and the panel route (M=100)
    ms = (4, 40, 100)
    xs = {m: synth.normal_fast(900 + m, m * k).reshape(m, k) for m in ms}
    X = {m: torch.from_numpy(xs[m]).to(dev) for m in ms}

    stream = torch.cuda.Stream()          # default priority; fresh scratch entry
    iters = 12
    outs = {m: [torch.full((m, n), float("nan"), device=dev) for _ in range(iters)] for m in ms}
    torch.cuda.synchronize()
    errors = []

    def worker(m):
        try:
            for i in range(iters):
                stt = qc.qgemm_raw(fmt, P, X[m], outs[m][i], m, n, k, stream=stream.cuda_stream)
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
        alone = torch.empty((m, n), device=dev)
        with torch.cuda.stream(stream):
            qc.qgemm(fmt, P, X[m], n, k, y=alone)
        torch.cuda.synchronize()
        want = alone.cpu().numpy()
        for i in range(iters):
            got = outs[m][i].cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, i)
        y64, wn = oracle.qgemm_f64(fmt, packed, xs[m], n, k)
        for r in range(m):
            ok, worst = oracle.within_contract(want[r], y64[r], wn, xs[m][r], 1e-4)
            assert ok, (m, r, worst)
