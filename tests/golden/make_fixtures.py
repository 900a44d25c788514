"""Writes the committed fixtures of this directory (run from the repository
root after `make -C oracle all ref`):

* synthetic_sha256.json -- SHA-256 of the seeded synthetic byte streams that
  the tests feed the GPU path at the BASELINE configs' full sizes (f32
  weights and activations from quixicore_hip.synth, and their q8_0 / q4_0 /
  int8 encodings by the oracle).  A change of generator, packer or quantizer
  shows up as a changed hash.
* reference_vectors.npz -- small inputs and the outputs of the reference's
  own compiled functions (oracle/_ref, built from the reference sources) on
  them: q8_0 / q4_0 packing, the x86 GEMV routes, qgemm, quantize_int8 and
  the dispatched int8_gemm.  tests/test_golden.py checks the oracle against
  them where the reference build is not available.
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for p in (os.path.join(ROOT, "quixicore-cpu_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)
HERE = os.path.dirname(os.path.abspath(__file__))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def streams():
    """(name, array) pairs of the full-size synthetic inputs."""
    import oracle
    from quixicore_hip import synth
    out = []
    w0 = synth.weights(0, 4096, 4096)
    out += [("c0_w_f32_4096x4096", w0), ("c0_w_q8_0", oracle.pack(oracle.Q8_0, w0)[1]),
            ("c0_x_f32_4096", synth.activations(0, 1, 4096))]
    w1 = synth.weights(1, 14336, 4096)
    out += [("c1_up_w_f32_14336x4096", w1), ("c1_up_w_q4_0", oracle.pack(oracle.Q4_0, w1)[1])]
    w1d = synth.weights(1, 4096, 14336)
    out += [("c1_down_w_f32_4096x14336", w1d),
            ("c1_down_w_q4_0", oracle.pack(oracle.Q4_0, w1d)[1]),
            ("c1_x_f32_4096", synth.activations(1, 1, 4096)),
            ("c1_x_f32_14336", synth.activations(1, 1, 14336))]
    out += [("c2_x_f32_32x4096", synth.activations(2, 32, 4096))]
    x3 = synth.activations_outliers_fast(3, 2048, 4096)
    st, xq, xs = oracle.quantize_int8(x3)
    out += [("c3_x_f32_2048x4096", x3), ("c3_x_codes", xq), ("c3_x_scales", xs)]
    for n, tid in ((4096, 3), (14336, 4)):
        st, wq, ws = oracle.quantize_int8(synth.weights(3, n, 4096, tensor_id=tid))
        out += [(f"c3_w_codes_{n}x4096", wq), (f"c3_w_scales_{n}", ws)]
    return out


def vectors():
    import oracle
    from quixicore_hip import synth
    ref = oracle.Reference()
    ref.set_threads(1)
    v = {}
    n, k, m = 24, 256, 5
    w = synth.weights(9, n, k)
    w[0, :32] = 0.0                                  # an all-zero block (q4_0: d = -0)
    w[1, 40] = 1e-9                                   # tiny values: subnormal fp16 scale
    w[1, 32:64] *= 1e-4
    x = synth.activations(9, m, k)
    v["w"], v["x"] = w, x
    for fmt, name in ((oracle.Q8_0, "q8_0"), (oracle.Q4_0, "q4_0")):
        st, packed = ref.pack(fmt, w)
        assert st == 0
        v[f"{name}_packed"] = packed
        v[f"{name}_gemv"] = ref.gemv(fmt, packed, x[0], n, k)
        v[f"{name}_qgemm"] = ref.qgemm(fmt, packed, x, n, k)
    v["q4_0_gemv_portable"] = ref.gemv(oracle.Q4_0, v["q4_0_packed"], x[0], n, k, portable=True)
    xo = synth.activations_outliers_fast(9, 7, 96)
    xo[2] = 0.0                                       # all-zero row: scale 0, codes 0
    xo[3, 5] = 127.5 / 127.0 * 3.0                    # near a tie
    st, codes, scales = ref.quantize_int8(xo)
    assert st == 0
    v["qi8_x"], v["qi8_codes"], v["qi8_scales"] = xo, codes, scales
    st, gcodes, gscales = ref.quantize_int8(xo, group_size=32)
    v["qi8_group32_codes"], v["qi8_group32_scales"] = gcodes, gscales
    rng = np.random.default_rng(9)
    wi = rng.integers(-128, 128, (13, 100), dtype=np.int8)
    xi = rng.integers(-128, 128, (6, 100), dtype=np.int8)
    wi[0, :] = -128
    xi[0, :] = -128
    wsc = rng.uniform(1e-4, 1e-2, 13).astype(np.float32)
    asc = rng.uniform(1e-3, 1e-1, 6).astype(np.float32)
    rs = wi.astype(np.int32).sum(axis=1).astype(np.int32)
    zp = rng.integers(-128, 128, 6).astype(np.int32)
    st, y = ref.int8_gemm(wi, xi, wsc, asc)
    st2, ya = ref.int8_gemm(wi, xi, wsc, asc, rs, zp, True)
    assert st == 0 and st2 == 0
    v.update(i8_w=wi, i8_x=xi, i8_ws=wsc, i8_as=asc, i8_rs=rs, i8_zp=zp, i8_y=y, i8_y_azp=ya)
    v["int8_gemm_variant"] = np.array(ref.variant())
    return v


def main():
    hashes = {name: {"sha256": sha(a), "dtype": str(a.dtype), "shape": list(a.shape)}
              for name, a in streams()}
    with open(os.path.join(HERE, "synthetic_sha256.json"), "w") as f:
        json.dump(hashes, f, indent=1, sort_keys=True)
        f.write("\n")
    np.savez_compressed(os.path.join(HERE, "reference_vectors.npz"), **vectors())


if __name__ == "__main__":
    main()
