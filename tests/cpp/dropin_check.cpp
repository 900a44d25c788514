// Exercises the C++ drop-in API (include/quixicore_cpu/*.h) the way a caller
// of the reference does: host std::vector buffers, synchronous calls,
// reference Status values.  Every input and output is written under argv[1]
// (raw little-endian arrays plus a manifest: "name dtype count" or
// "name status value" per line); tests/test_gpu_dropin.py checks them
// against the CPU oracle.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/qgemv.h"
#include "quixicore_cpu/qgemv_w8a8.h"
#include "quixicore_cpu/quantization.h"
#include "quixicore_cpu/workspace.h"

namespace qc = quixicore_cpu;

namespace {

struct Sink {
  std::string dir;
  FILE* manifest = nullptr;

  template <class T>
  void put(const std::string& name, const std::vector<T>& v, const char* dtype) {
    FILE* f = std::fopen((dir + "/" + name + ".bin").c_str(), "wb");
    if (f == nullptr) return;
    if (!v.empty()) std::fwrite(v.data(), sizeof(T), v.size(), f);
    std::fclose(f);
    std::fprintf(manifest, "%s %s %zu\n", name.c_str(), dtype, v.size());
  }
  void status(const std::string& name, qc::Status s) {
    std::fprintf(manifest, "%s status %d\n", name.c_str(), static_cast<int>(s));
  }
};

// xorshift32 values in [-1, 1) times scale.
std::vector<float> values(uint32_t seed, size_t n, float scale) {
  std::vector<float> v(n);
  uint32_t s = seed | 1u;
  for (size_t i = 0; i < n; ++i) {
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    v[i] = (static_cast<float>(s >> 8) * (2.0f / 16777216.0f) - 1.0f) * scale;
  }
  return v;
}

std::vector<int8_t> codes(uint32_t seed, size_t n) {
  std::vector<int8_t> v(n);
  uint32_t s = seed | 1u;
  for (size_t i = 0; i < n; ++i) {
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    v[i] = static_cast<int8_t>(static_cast<int>(s >> 24) - 128);
  }
  return v;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: dropin_check <output dir>\n");
    return 2;
  }
  Sink out{argv[1], std::fopen((std::string(argv[1]) + "/manifest.txt").c_str(), "w")};
  if (out.manifest == nullptr) return 2;
  const long long n = 96, k = 256, m = 5;

  // pack, qgemv, qgemm, fused projections, w8a8 GEMV: both formats
  for (int f = 0; f < 2; ++f) {
    const qc::QuantFormat fmt = f == 0 ? qc::QuantFormat::kQ8_0 : qc::QuantFormat::kQ4_0;
    const std::string p = f == 0 ? "q8_0_" : "q4_0_";
    size_t bytes = 0;
    out.status(p + "packed_size", qc::qgemv_packed_size(fmt, n, k, &bytes));
    std::vector<float> w = values(11 + f, n * k, 0.05f), w2 = values(21 + f, n * k, 0.05f);
    std::vector<uint8_t> pw(bytes), pw2(bytes);
    out.status(p + "pack", qc::qgemv_pack(fmt, w.data(), n, k, pw.data()));
    out.status(p + "pack2", qc::qgemv_pack(fmt, w2.data(), n, k, pw2.data()));
    out.put(p + "w", w, "f32");
    out.put(p + "w2", w2, "f32");
    out.put(p + "packed", pw, "u8");
    out.put(p + "packed2", pw2, "u8");
    std::vector<float> x = values(31 + f, m * k, 1.0f);
    out.put(p + "x", x, "f32");
    std::vector<float> y(n), y2(n), ym(m * n), act(n);
    out.status(p + "qgemv", qc::qgemv(fmt, pw.data(), x.data(), y.data(), n, k));
    out.put(p + "qgemv_y", y, "f32");
    out.status(p + "qgemm", qc::qgemm(fmt, pw.data(), x.data(), ym.data(), m, n, k));
    out.put(p + "qgemm_y", ym, "f32");
    out.status(p + "up_gate",
               qc::qgemv_up_gate(fmt, pw.data(), pw2.data(), x.data(), y.data(), y2.data(), n, k));
    out.put(p + "up", y, "f32");
    out.put(p + "gate", y2, "f32");
    out.status(p + "up_gate_gelu", qc::qgemv_up_gate_activation(fmt, pw.data(), pw2.data(),
                                                                x.data(), act.data(), n, k, true));
    out.put(p + "act_gelu", act, "f32");
    out.status(p + "up_gate_silu", qc::qgemv_up_gate_activation(fmt, pw.data(), pw2.data(),
                                                                x.data(), act.data(), n, k, false));
    out.put(p + "act_silu", act, "f32");
    std::vector<float> q(n), kk(n / 2), vv(n / 2);
    out.status(p + "qkv", qc::qgemv_qkv(fmt, pw.data(), pw2.data(), pw2.data() + bytes / 2,
                                        x.data(), q.data(), kk.data(), vv.data(), n, n / 2, k));
    out.put(p + "qkv_q", q, "f32");
    out.put(p + "qkv_k", kk, "f32");
    out.put(p + "qkv_v", vv, "f32");
    // RoPE seam: 6 query heads and 3 kv heads of 16, cache slot 1 of 3 at position 2
    {
      const long long hd = 16, slots = 3, max_pos = 4;
      std::vector<float> cs = values(61 + f, max_pos * hd / 2, 1.0f);
      std::vector<float> sn = values(71 + f, max_pos * hd / 2, 1.0f);
      std::vector<float> rq(n), kc = values(81, slots * n / 2, 9.0f), vc = values(82, slots * n / 2, 9.0f);
      out.put(p + "rope_cos", cs, "f32");
      out.put(p + "rope_sin", sn, "f32");
      out.put(p + "rope_kc0", kc, "f32");
      out.put(p + "rope_vc0", vc, "f32");
      out.status(p + "qkv_rope", qc::qgemv_qkv_rope_kv(fmt, pw.data(), pw2.data(),
                                                        pw2.data() + bytes / 2, x.data(), cs.data(),
                                                        sn.data(), rq.data(), kc.data(), vc.data(),
                                                        n / hd, n / 2 / hd, hd, k, slots, max_pos,
                                                        2, 1));
      out.put(p + "rope_q", rq, "f32");
      out.put(p + "rope_kc", kc, "f32");
      out.put(p + "rope_vc", vc, "f32");
      out.status(p + "qkv_rope_badpos", qc::qgemv_qkv_rope_kv(
                                            fmt, pw.data(), pw2.data(), pw2.data(), x.data(),
                                            cs.data(), sn.data(), rq.data(), kc.data(), vc.data(),
                                            n / hd, n / 2 / hd, hd, k, slots, max_pos, 4, 1));
    }
    out.status(p + "w8a8", qc::qgemv_w8a8(fmt, pw.data(), x.data(), y.data(), n, k));
    out.put(p + "w8a8_y", y, "f32");

    // prepared weights with an explicit workspace: M = 1, small M, M >= 64
    qc::CpuPackedWeights prepared;
    out.status(p + "prepare", prepared.prepare(fmt, pw.data(), n, k));
    qc::Workspace ws;
    out.status(p + "prepacked_gemv", qc::qgemv_prepacked(prepared, x.data(), y.data(), &ws));
    out.put(p + "prepacked_gemv_y", y, "f32");
    out.status(p + "prepacked_m5", qc::qgemm_prepacked(prepared, x.data(), ym.data(), m, &ws));
    out.put(p + "prepacked_m5_y", ym, "f32");
    std::vector<float> xl = values(41 + f, 70 * k, 1.0f), yl(70 * n);
    out.put(p + "xl", xl, "f32");
    out.status(p + "prepacked_m70", qc::qgemm_prepacked(prepared, xl.data(), yl.data(), 70, &ws));
    out.put(p + "prepacked_m70_y", yl, "f32");
  }

  // validation without touching memory
  float dummy = 0.f;
  out.status("bad_k", qc::qgemv(qc::QuantFormat::kQ8_0, &dummy, &dummy, &dummy, 4, 33));
  out.status("null_y", qc::qgemv(qc::QuantFormat::kQ8_0, &dummy, &dummy, nullptr, 4, 32));

  // quantize_int8, per row and per 32-group
  {
    std::vector<float> x = values(51, 4 * 256, 3.0f);
    out.put("quant_x", x, "f32");
    for (long long g : {0LL, 32LL}) {
      std::vector<int8_t> c(4 * 256);
      std::vector<float> s(4 * (256 / (g == 0 ? 256 : g)));
      const std::string p = "quant_g" + std::to_string(g);
      out.status(p, qc::quantize_int8(x.data(), c.data(), s.data(), 4, 256, g));
      out.put(p + "_codes", c, "i8");
      out.put(p + "_scales", s, "f32");
    }
  }

  // int8 GEMM, plain and with activation zero points
  {
    const long long gm = 5, gn = 7, gk = 64;
    std::vector<int8_t> w = codes(61, gn * gk), x = codes(62, gm * gk);
    std::vector<float> ws = values(63, gn, 0.01f), as = values(64, gm, 0.1f);
    for (float& v : ws) v = std::fabs(v) + 1e-3f;
    for (float& v : as) v = std::fabs(v) + 1e-3f;
    std::vector<int32_t> rs(gn);
    for (long long r = 0; r < gn; ++r) {
      int32_t t = 0;
      for (long long i = 0; i < gk; ++i) t += w[r * gk + i];
      rs[r] = t;
    }
    std::vector<int> zp = {3, -2, 0, 7, -128};
    out.put("i8_w", w, "i8");
    out.put("i8_x", x, "i8");
    out.put("i8_ws", ws, "f32");
    out.put("i8_as", as, "f32");
    out.put("i8_rs", rs, "i32");
    out.put("i8_zp", zp, "i32");
    std::vector<float> y(gm * gn);
    out.status("int8_gemm", qc::int8_gemm(w.data(), x.data(), ws.data(), as.data(), nullptr,
                                          nullptr, y.data(), gm, gn, gk));
    out.put("int8_gemm_y", y, "f32");
    out.status("w8a8", qc::qgemm_w8a8(w.data(), x.data(), ws.data(), as.data(), y.data(), gm, gn,
                                      gk));
    out.put("w8a8_y", y, "f32");
    out.status("w8a8_azp", qc::qgemm_w8a8_azp(w.data(), x.data(), ws.data(), as.data(), rs.data(),
                                              zp.data(), y.data(), gm, gn, gk));
    out.put("w8a8_azp_y", y, "f32");
  }

  // rms_norm_add_quant_int8 with one non-finite weight: its group keeps the
  // caller's sentinels, everything else is written, status kInvalidArgument
  {
    const long long rows = 3, hidden = 256, group = 32;
    std::vector<float> x = values(71, rows * hidden, 2.0f), r = values(72, rows * hidden, 2.0f);
    std::vector<float> w = values(73, hidden, 1.0f);
    out.put("norm_x", x, "f32");
    out.put("norm_r", r, "f32");
    out.put("norm_w_ok", w, "f32");
    std::vector<int8_t> c(rows * hidden, 0x5A);
    std::vector<float> ro(rows * hidden, 0.f), s(rows * hidden / group, -7.0f);
    out.status("norm_ok", qc::rms_norm_add_quant_int8(x.data(), r.data(), w.data(), c.data(),
                                                      ro.data(), s.data(), rows, hidden, 1e-5f,
                                                      group));
    out.put("norm_ok_codes", c, "i8");
    out.put("norm_ok_resid", ro, "f32");
    out.put("norm_ok_scales", s, "f32");
    w[40] = INFINITY;
    out.put("norm_w_bad", w, "f32");
    std::fill(c.begin(), c.end(), static_cast<int8_t>(0x5A));
    std::fill(ro.begin(), ro.end(), 0.f);
    std::fill(s.begin(), s.end(), -7.0f);
    out.status("norm_bad", qc::rms_norm_add_quant_int8(x.data(), r.data(), w.data(), c.data(),
                                                       ro.data(), s.data(), rows, hidden, 1e-5f,
                                                       group));
    out.put("norm_bad_codes", c, "i8");
    out.put("norm_bad_resid", ro, "f32");
    out.put("norm_bad_scales", s, "f32");
    // in place: residual_out is the residual array itself
    std::vector<float> r2 = r;
    w[40] = 0.5f;
    out.put("norm_w_inplace", w, "f32");
    out.status("norm_inplace", qc::rms_norm_add_quant_int8(x.data(), r2.data(), w.data(), c.data(),
                                                           r2.data(), s.data(), rows, hidden,
                                                           1e-5f, 0));
    out.put("norm_inplace_codes", c, "i8");
    out.put("norm_inplace_resid", r2, "f32");
    out.put("norm_inplace_scales", std::vector<float>(s.begin(), s.begin() + rows), "f32");
  }

  // asymmetric int8 round trip
  {
    std::vector<float> x = values(81, 3 * 200, 4.0f);
    for (float& v : x) v += 1.5f;
    out.put("asym_x", x, "f32");
    std::vector<int8_t> c(3 * 200);
    std::vector<float> s(3), d(3 * 200);
    std::vector<int> z(3);
    out.status("asym", qc::quantize_int8_asymmetric(x.data(), c.data(), s.data(), z.data(), 3, 200));
    out.put("asym_codes", c, "i8");
    out.put("asym_scales", s, "f32");
    out.put("asym_zps", z, "i32");
    out.status("asym_deq", qc::dequantize_int8_asymmetric(c.data(), s.data(), z.data(), d.data(),
                                                          3, 200));
    out.put("asym_deq_y", d, "f32");
  }
  std::fclose(out.manifest);
  return 0;
}
