"""Checks one run of tests/cpp/storage_scenarios.h (the prepared storage
projections over canonical int8 weights) against the f64 restatement in
oracle/oracle.py.  Used on the reference's run (tests/test_oracle.py, which
pins the restatement) and on this library's run (tests/test_gpu_canonical.py).

Bounds, per output (contract tolerance TOL after normalising by
||x_row||_2 * ||w_hat_row||_2, as for every f32 projection of this path):
  * plain projection y:      |y - y64| <= TOL * ||x|| * ||w_hat_n||
  * bias + activation:       the same times max(1.2, 2|v| + 1) (the
                             activation's slope bound; ReLU^2 grows as 2v)
  * SiLU(gate) * up:         TOL * ||x|| * (1.1 |up| ||w_gate|| + |SiLU(gate)| ||w_up||)
  * RoPE pair:               TOL * ||x|| * (||w_a|| + ||w_b||) * (|c| + |s|)
plus, for 16-bit outputs, half a unit in the last place of the stored type.
Cache elements outside the written slot must keep their 0x5a fill.
"""
import os

import numpy as np

TOL = 1e-4
K = 256
SPECS = {"A": (72, K, 0, False), "B": (72, K, 64, True), "C": (72, K, 32, False),
         "D": (40, 40, 0, False), "E": (24, 96, 48, True)}
FILL32 = np.frombuffer(b"\x5a" * 4, np.float32)[0]
FILL16 = 0x5a5a


def load(directory):
    status, data = {}, {}
    for line in open(os.path.join(directory, "manifest.txt")):
        name, kind, value = line.split()
        if kind == "status":
            status[name] = int(value)
        else:
            raw = np.fromfile(os.path.join(directory, name + ".bin"), dtype=np.uint8)
            data[name] = (kind, raw)
    return status, data


def _f32(entry):
    kind, raw = entry
    if kind == "f32":
        return raw.view(np.float32)
    bits = raw.view(np.uint16)
    if kind == "f16":
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _ulp_half(kind, ref):
    if kind == "f16":
        return np.abs(ref) * 2.0 ** -11 + 2.0 ** -25
    if kind == "bf16":
        return np.abs(ref) * 2.0 ** -8 + 2.0 ** -134
    return 0.0


def _weights(oracle, data, name, rows, cols, groups, affine):
    codes = data[name + ".codes"][1].view(np.int8)
    scales = data[name + ".scales"][1].view(np.float32)
    zeros = data[name + ".zeros"][1].view(np.float32) if affine else None
    return oracle.cint8_dequant(codes, scales, zeros, rows, cols, groups)


def check(oracle, directory):
    """Returns (statuses, list of failure strings)."""
    status, data = load(directory)
    bad = []

    def expect(name, ok, detail=""):
        if not ok:
            bad.append(f"{name} {detail}")

    def plain(name, x, w, out):
        kind = data[out][0]
        y = _f32(data[out]).astype(np.float64)
        y64, wn = oracle.cint8_project_f64(x, w)
        y64 = y64.reshape(-1)
        xn = np.repeat(np.linalg.norm(np.asarray(x, np.float64).reshape(len(x), -1), axis=1), w.shape[0])
        bound = TOL * xn * np.tile(wn, len(x)) + _ulp_half(kind, y64)
        expect(out, y.shape == y64.shape and np.all(np.abs(y - y64) <= bound),
               f"max excess {np.max(np.abs(y - y64) - bound) if y.shape == y64.shape else 'shape'}")

    for p, (rows, cols, group, affine) in SPECS.items():
        groups = cols // group if group else 1
        expect(p + "_prepare", status.get(p + "_prepare") == 0)
        w = _weights(oracle, data, p, rows, cols, groups, affine)
        for m in (1, 3, 5, 16):
            x = _f32(data[f"{p}_m{m}.x"]).reshape(m, cols)
            for ty in ("00", "10", "22", "01"):
                c = f"{p}_m{m}_{ty}"
                expect(c, status.get(c) == 0, f"status {status.get(c)}")
                plain(c, x, w, c + ".y")
            expect(f"{p}_m{m}_prepacked", status.get(f"{p}_m{m}_prepacked") == 0)
            plain(f"{p}_m{m}_prepacked", x, w, f"{p}_m{m}_prepacked.y")
        x = _f32(data[f"{p}_epi.x"]).reshape(2, cols)
        bias = _f32(data[f"{p}_epi.bias"]).astype(np.float64)
        y64, wn = oracle.cint8_project_f64(x, w)
        xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
        for a in range(5):
            c = f"{p}_epi{a}"
            expect(c, status.get(c) == 0, f"status {status.get(c)}")
            v = y64 + (bias if a % 2 else 0.0)
            want = oracle.linear_activation_f64(v, a)
            y = _f32(data[c + ".y"]).reshape(2, rows).astype(np.float64)
            bound = TOL * xn * wn[None, :] * np.maximum(1.2, 2 * np.abs(v) + 1) + 1e-6 * np.abs(want)
            expect(c, np.all(np.abs(y - want) <= bound), f"max excess {np.max(np.abs(y - want) - bound)}")
        x1 = _f32(data[f"{p}_gemv.x"]).reshape(1, cols)
        expect(p + "_gemv", status.get(p + "_gemv") == 0)
        plain(p + "_gemv", x1, w, p + "_gemv.y")

    for affine, p in ((0, "ps"), (1, "pa")):
        groups = K // 64 if affine else 1
        ws = {}
        for nm, rows in (("g", 96), ("u", 96), ("q", 64), ("k", 32), ("v", 32)):
            expect(p + nm + "_prepare", status.get(p + nm + "_prepare") == 0)
            ws[nm] = _weights(oracle, data, p + nm, rows, K, groups, affine)
        for m in (1, 3):
            c = f"{p}_gu_m{m}"
            x = _f32(data[c + ".x"]).reshape(m, K)
            for sub in ("", "_swiglu", "_qkv"):
                expect(c + sub, status.get(c + sub) == 0, f"status {status.get(c + sub)}")
            plain(c, x, ws["g"], c + ".gate")
            plain(c, x, ws["u"], c + ".up")
            g64, gn = oracle.cint8_project_f64(x, ws["g"])
            u64, un = oracle.cint8_project_f64(x, ws["u"])
            silu = g64 / (1.0 + np.exp(-g64))
            want = silu * u64
            xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
            bound = TOL * xn * (1.1 * np.abs(u64) * gn + np.abs(silu) * un) + 1e-6 * np.abs(want)
            y = _f32(data[c + "_swiglu.y"]).reshape(m, 96)
            expect(c + "_swiglu", np.all(np.abs(y - want) <= bound), f"max excess {np.max(np.abs(y - want) - bound)}")
            for nm in ("q", "k", "v"):
                plain(c + "_qkv", x, ws[nm], c + "_qkv." + nm)
        x = _f32(data[p + "_rope.x"]).reshape(1, K)
        cs = _f32(data[p + "_rope.cos"]).reshape(4, 8)[2].astype(np.float64)
        sn = _f32(data[p + "_rope.sin"]).reshape(4, 8)[2].astype(np.float64)
        xn = np.linalg.norm(x.astype(np.float64))

        def rotated(nm, heads):
            y64, wn = oracle.cint8_project_f64(x, ws[nm])
            a, b = y64.reshape(heads, 2, 8)[:, 0], y64.reshape(heads, 2, 8)[:, 1]
            na, nb = wn.reshape(heads, 2, 8)[:, 0], wn.reshape(heads, 2, 8)[:, 1]
            out = np.stack([a * cs - b * sn, b * cs + a * sn], 1).reshape(-1)
            bnd = TOL * xn * np.repeat((na + nb) * (np.abs(cs) + np.abs(sn)), 1, axis=0)
            return out, np.stack([bnd, bnd], 1).reshape(-1)

        for ct in ("0", "1"):
            for sl in ("_slot1", "_noslot"):
                c = f"{p}_rope_{ct}{sl}"
                expect(c, status.get(c) == 0, f"status {status.get(c)}")
                want, bnd = rotated("q", 4)
                y = _f32(data[c + ".q"]).astype(np.float64)
                expect(c + ".q", np.all(np.abs(y - want) <= bnd), f"max excess {np.max(np.abs(y - want) - bnd)}")
                for cache, nm in ((".kc", "k"), (".vc", "v")):
                    kind, raw = data[c + cache]
                    vals = _f32(data[c + cache]).astype(np.float64)
                    fill = raw.view(np.float32) == FILL32 if kind == "f32" else raw.view(np.uint16) == FILL16
                    keep = np.ones(96, bool)
                    if sl == "_slot1":
                        keep[32:64] = False
                        if nm == "k":
                            want, bnd = rotated("k", 2)
                        else:
                            y64, wn = oracle.cint8_project_f64(x, ws["v"])
                            want, bnd = y64.reshape(-1), TOL * xn * wn
                        got = vals[32:64]
                        bnd = bnd + _ulp_half(kind, want)
                        expect(c + cache, np.all(np.abs(got - want) <= bnd),
                               f"max excess {np.max(np.abs(got - want) - bnd)}")
                    expect(c + cache + " fill", np.all(fill[keep]))
    return status, bad
