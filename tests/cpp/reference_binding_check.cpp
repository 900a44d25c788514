// Drives the reference-side binding (tests/cpp/reference_binding.h) the way
// the reference's dispatch would call it: host std::vector buffers,
// synchronous calls, statuses returned unchanged.
//
// usage: reference_binding_check <dir>
// Reads the operands tests/test_gpu_reference_binding.py wrote into <dir>
// (dims.txt "n k m", q4.bin, q8.bin, x.bin, xq.bin, w8.bin, x8.bin, ws.bin,
// as.bin, rs.bin, zp.bin), writes each output as <name>.bin and every status
// as "name value" lines of status.txt.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <string>
#include <vector>

#include "reference_binding.h"

namespace hb = quixicore_cpu::hip_gfx950;

namespace {

std::string g_dir;
FILE* g_status = nullptr;

template <class T>
std::vector<T> load(const char* name) {
  std::vector<T> v;
  FILE* f = std::fopen((g_dir + "/" + name).c_str(), "rb");
  if (f == nullptr) return v;
  std::fseek(f, 0, SEEK_END);
  const long bytes = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  v.resize(static_cast<std::size_t>(bytes) / sizeof(T));
  if (!v.empty() && std::fread(v.data(), sizeof(T), v.size(), f) != v.size()) v.clear();
  std::fclose(f);
  return v;
}

template <class T>
void save(const std::string& name, const std::vector<T>& v) {
  FILE* f = std::fopen((g_dir + "/" + name + ".bin").c_str(), "wb");
  if (f == nullptr) return;
  if (!v.empty()) std::fwrite(v.data(), sizeof(T), v.size(), f);
  std::fclose(f);
}

void status(const char* name, int value) { std::fprintf(g_status, "%s %d\n", name, value); }

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: reference_binding_check <dir>\n");
    return 2;
  }
  g_dir = argv[1];
  long long n = 0, k = 0, m = 0;
  FILE* dims = std::fopen((g_dir + "/dims.txt").c_str(), "r");
  if (dims == nullptr || std::fscanf(dims, "%lld %lld %lld", &n, &k, &m) != 3) return 2;
  std::fclose(dims);
  g_status = std::fopen((g_dir + "/status.txt").c_str(), "w");
  if (g_status == nullptr) return 2;

  status("available", hb::available() ? 1 : 0);
  unsetenv("QUIXICORE_CPU_QGEMV_VARIANT");
  status("selected_default", hb::selected("QUIXICORE_CPU_QGEMV_VARIANT") ? 1 : 0);
  setenv("QUIXICORE_CPU_QGEMV_VARIANT", "ref", 1);
  status("selected_ref", hb::selected("QUIXICORE_CPU_QGEMV_VARIANT") ? 1 : 0);
  setenv("QUIXICORE_CPU_QGEMV_VARIANT", "hip_gfx950", 1);
  status("selected_named", hb::selected("QUIXICORE_CPU_QGEMV_VARIANT") ? 1 : 0);
  unsetenv("QUIXICORE_CPU_QGEMV_VARIANT");

  const std::vector<uint8_t> q4 = load<uint8_t>("q4.bin"), q8 = load<uint8_t>("q8.bin");
  const std::vector<float> x = load<float>("x.bin"), xq = load<float>("xq.bin");
  const std::vector<int8_t> w8 = load<int8_t>("w8.bin"), x8 = load<int8_t>("x8.bin");
  const std::vector<float> ws = load<float>("ws.bin"), as = load<float>("as.bin");
  const std::vector<int32_t> rs = load<int32_t>("rs.bin");
  const std::vector<int> zp = load<int>("zp.bin");
  if (x.size() != static_cast<std::size_t>(m * k) || w8.size() != static_cast<std::size_t>(n * k))
    return 2;

  // qgemv / qgemm, both formats
  for (int f = 0; f < 2; ++f) {
    const std::vector<uint8_t>& p = f == 0 ? q8 : q4;
    const std::string pre = f == 0 ? "q8_0_" : "q4_0_";
    std::vector<float> y(n, 7.0f), ym(m * n, 7.0f);
    status((pre + "qgemv").c_str(), hb::qgemv(f, p.data(), x.data(), y.data(), n, k));
    save(pre + "qgemv", y);
    status((pre + "qgemm").c_str(), hb::qgemm(f, p.data(), x.data(), ym.data(), m, n, k));
    save(pre + "qgemm", ym);
  }
  // validation results pass through unchanged, outputs untouched
  {
    std::vector<float> y(n, 7.0f);
    status("qgemv_bad_format", hb::qgemv(7, q4.data(), x.data(), y.data(), n, k));
    status("qgemv_bad_k", hb::qgemv(1, q4.data(), x.data(), y.data(), n, 33));
    status("qgemv_null_x", hb::qgemv(1, q4.data(), nullptr, y.data(), n, k));
    status("qgemm_null_before_format", hb::qgemm(9, nullptr, x.data(), y.data(), 1, n, k));
    save("untouched_qgemv", y);
  }
  // quantize_int8 per row and in groups of 128, then a non-finite x
  {
    std::vector<int8_t> codes(xq.size(), 5);
    std::vector<float> scales(m, 7.0f), gscales(m * (k / 128), 7.0f);
    status("quantize_rows", hb::quantize_int8(xq.data(), codes.data(), scales.data(), m, k, 0));
    save("quantize_codes", codes);
    save("quantize_scales", scales);
    std::vector<int8_t> gcodes(xq.size(), 5);
    status("quantize_groups",
           hb::quantize_int8(xq.data(), gcodes.data(), gscales.data(), m, k, 128));
    save("quantize_group_codes", gcodes);
    save("quantize_group_scales", gscales);
    std::vector<float> bad = xq;
    bad[k + 3] = std::numeric_limits<float>::infinity();
    std::vector<int8_t> c2(xq.size(), 5);
    std::vector<float> s2(m, 7.0f);
    status("quantize_nonfinite", hb::quantize_int8(bad.data(), c2.data(), s2.data(), m, k, 0));
    save("untouched_codes", c2);
    save("untouched_scales", s2);
    status("quantize_bad_group", hb::quantize_int8(xq.data(), c2.data(), s2.data(), m, k, 100));
  }
  // int8_gemm symmetric and with the zero-point correction, then a NaN scale
  {
    std::vector<float> y(m * n, 7.0f), ya(m * n, 7.0f);
    status("int8_gemm", hb::int8_gemm(w8.data(), x8.data(), ws.data(), as.data(), nullptr,
                                      nullptr, y.data(), m, n, k, false));
    save("int8_gemm", y);
    status("int8_gemm_azp", hb::int8_gemm(w8.data(), x8.data(), ws.data(), as.data(), rs.data(),
                                          zp.data(), ya.data(), m, n, k, true));
    save("int8_gemm_azp", ya);
    std::vector<float> bad = ws;
    bad[3] = std::nanf("");
    std::vector<float> yb(m * n, 7.0f);
    status("int8_gemm_nan_scale", hb::int8_gemm(w8.data(), x8.data(), bad.data(), as.data(),
                                                nullptr, nullptr, yb.data(), m, n, k, false));
    save("untouched_int8", yb);
    status("int8_gemm_asym_null", hb::int8_gemm(w8.data(), x8.data(), ws.data(), as.data(),
                                                nullptr, nullptr, yb.data(), m, n, k, true));
    status("int8_gemm_bad_shape", hb::int8_gemm(w8.data(), x8.data(), ws.data(), as.data(),
                                                nullptr, nullptr, yb.data(), 0, n, k, false));
  }
  std::fclose(g_status);
  return 0;
}
