// Prepared storage projections over canonical int8 weights -- TEST
// INFRASTRUCTURE ONLY.  One scenario list, compiled twice against the same
// C++ API (include/quixicore_cpu/qgemm.h:32-101): into oracle/_ref with the
// reference's own headers and library (oracle/ref_shim.cpp,
// qcref_storage_scenarios), and into tests/cpp/storage_check.cpp with this
// repository's drop-in headers and libquixicore_hip.so.  Both write every
// status and output under a directory; tests/test_gpu_canonical.py compares
// the two runs (statuses equal, outputs within the contract) and both against
// the f64 restatement in oracle/oracle.py.
//
// Inputs are deterministic (xorshift32) and exactly representable in f16 and
// bf16 (multiples of 1/64 below 2 in magnitude), so each 16-bit activation
// case is the f32 case's data in another storage type.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/quant_import.h"

namespace storage_scenarios {

namespace qc = quixicore_cpu;

struct Sink {
  std::string dir;
  FILE* manifest = nullptr;
  explicit Sink(const char* d) : dir(d) {
    manifest = std::fopen((dir + "/manifest.txt").c_str(), "w");
  }
  ~Sink() {
    if (manifest) std::fclose(manifest);
  }
  void status(const std::string& name, qc::Status s) {
    if (manifest) std::fprintf(manifest, "%s status %d\n", name.c_str(), static_cast<int>(s));
  }
  void data(const std::string& name, const void* p, size_t bytes, const char* dtype) {
    FILE* f = std::fopen((dir + "/" + name + ".bin").c_str(), "wb");
    if (f == nullptr) return;
    if (bytes) std::fwrite(p, 1, bytes, f);
    std::fclose(f);
    if (manifest) std::fprintf(manifest, "%s %s %zu\n", name.c_str(), dtype, bytes);
  }
};

inline uint32_t next(uint32_t* s) {
  *s ^= *s << 13;
  *s ^= *s >> 17;
  *s ^= *s << 5;
  return *s;
}

// k / 64 for k in [-127, 127]: exact in f32, f16 and bf16.
inline std::vector<float> activations(uint32_t seed, size_t n) {
  std::vector<float> v(n);
  uint32_t s = seed | 1u;
  for (auto& e : v) e = static_cast<float>(static_cast<int>(next(&s) % 255u) - 127) / 64.0f;
  return v;
}

inline uint16_t bf16_bits(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return static_cast<uint16_t>(b >> 16);
}

// Exact for zero and for normal f16 values with at most 11 significant bits.
inline uint16_t f16_bits(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  const uint32_t sign = (b >> 16) & 0x8000u;
  if ((b & 0x7fffffffu) == 0) return static_cast<uint16_t>(sign);
  const int e = static_cast<int>((b >> 23) & 0xff) - 127 + 15;
  return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | ((b >> 13) & 0x3ffu));
}

struct Tensor {
  qc::CanonicalQuantTensor t;
  std::vector<int8_t> codes;
};

// int8 canonical tensor: scale_mode kChannel (groups == 1) or kGroup.
inline qc::CanonicalQuantTensor int8_tensor(uint32_t seed, long long rows, long long cols,
                                            bool affine, long long group) {
  qc::CanonicalQuantTensor t;
  t.metadata.layout =
      affine ? qc::CanonicalQuantLayout::kInt8Affine : qc::CanonicalQuantLayout::kInt8Symmetric;
  t.metadata.logical_rows = rows;
  t.metadata.logical_columns = cols;
  t.metadata.group_size = group > 0 ? group : cols;
  t.metadata.scale_mode = group > 0 ? qc::QuantScaleMode::kGroup : qc::QuantScaleMode::kChannel;
  t.metadata.scale_encoding = qc::QuantScaleEncoding::kFP32;
  const long long groups = group > 0 ? cols / group : 1;
  t.metadata.scale_count = static_cast<size_t>(rows * groups);
  uint32_t s = seed | 1u;
  t.data.resize(static_cast<size_t>(rows * cols));
  for (auto& c : t.data) c = static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(next(&s) % 255u) - 127));
  for (long long i = 0; i < rows * groups; ++i)
    t.scales.push_back(static_cast<float>(1 + next(&s) % 1000u) * 1e-5f);
  if (affine) {
    t.metadata.zero_point_mode = qc::QuantZeroPointMode::kInteger;
    t.metadata.zero_point_count = t.metadata.scale_count;
    for (long long i = 0; i < rows * groups; ++i)
      t.zero_points.push_back(static_cast<float>(static_cast<int>(next(&s) % 21u) - 10));
  }
  return t;
}

inline qc::FloatStorageInput in_of(const std::vector<float>& f32, std::vector<uint16_t>* bits,
                                   qc::FloatStorageType type) {
  if (type == qc::FloatStorageType::kF32)
    return {f32.data(), type, static_cast<long long>(f32.size())};
  bits->resize(f32.size());
  for (size_t i = 0; i < f32.size(); ++i)
    (*bits)[i] = type == qc::FloatStorageType::kF16 ? f16_bits(f32[i]) : bf16_bits(f32[i]);
  return {bits->data(), type, static_cast<long long>(f32.size())};
}

// An output buffer of `count` elements of `type`, pre-filled with a pattern.
struct Out {
  std::vector<uint8_t> bytes;
  qc::FloatStorageType type;
  long long count;
  Out(qc::FloatStorageType t, long long n)
      : bytes(static_cast<size_t>(n) * (t == qc::FloatStorageType::kF32 ? 4 : 2), 0x5a),
        type(t),
        count(n) {}
  qc::FloatStorageOutput view() { return {bytes.data(), type, count}; }
  const char* dtype() const {
    return type == qc::FloatStorageType::kF32 ? "f32" : type == qc::FloatStorageType::kF16 ? "f16" : "bf16";
  }
};

inline void put(Sink& sink, const std::string& name, const Out& o) {
  sink.data(name, o.bytes.data(), o.bytes.size(), o.dtype());
}

// The whole scenario list.  Names are "<case>" for statuses and
// "<case>.<output>" for data.
inline void run(Sink& sink) {
  using FT = qc::FloatStorageType;
  const long long K = 256;
  // weights: (A) symmetric channel scales, (B) affine groups of 64,
  // (C) symmetric groups of 32, (D) symmetric K = 40 (no 16-column chunks),
  // (E) affine groups of 48 (not a power of two)
  struct Spec {
    const char* name;
    long long rows, cols, group;
    bool affine;
  };
  const Spec specs[] = {{"A", 72, K, 0, false}, {"B", 72, K, 64, true}, {"C", 72, K, 32, false},
                        {"D", 40, 40, 0, false}, {"E", 24, 96, 48, true}};
  uint32_t seed = 11;
  for (const Spec& sp : specs) {
    const qc::CanonicalQuantTensor t = int8_tensor(seed++, sp.rows, sp.cols, sp.affine, sp.group);
    const std::string p = sp.name;
    sink.data(p + ".codes", t.data.data(), t.data.size(), "i8");
    sink.data(p + ".scales", t.scales.data(), t.scales.size() * 4, "f32");
    if (sp.affine) sink.data(p + ".zeros", t.zero_points.data(), t.zero_points.size() * 4, "f32");
    qc::CpuPackedWeights w;
    sink.status(p + "_prepare", w.prepare(t, qc::CpuPanelLayout::kPortableRows1));
    for (long long m : {1LL, 3LL, 5LL, 16LL}) {
      const std::vector<float> x = activations(seed++, static_cast<size_t>(m * sp.cols));
      sink.data(p + "_m" + std::to_string(m) + ".x", x.data(), x.size() * 4, "f32");
      const FT types[][2] = {{FT::kF32, FT::kF32}, {FT::kF16, FT::kF32}, {FT::kBF16, FT::kBF16},
                             {FT::kF32, FT::kF16}};
      for (const auto& ty : types) {
        std::vector<uint16_t> xb;
        Out y(ty[1], m * sp.rows);
        const std::string c = p + "_m" + std::to_string(m) + "_" + std::to_string(static_cast<int>(ty[0])) +
                              std::to_string(static_cast<int>(ty[1]));
        sink.status(c, qc::qgemm_prepacked_storage(w, in_of(x, &xb, ty[0]), y.view(), m));
        put(sink, c + ".y", y);
      }
      std::vector<float> yf(static_cast<size_t>(m * sp.rows), -1.0f);
      sink.status(p + "_m" + std::to_string(m) + "_prepacked",
                  qc::qgemm_prepacked(w, x.data(), yf.data(), m));
      sink.data(p + "_m" + std::to_string(m) + "_prepacked.y", yf.data(), yf.size() * 4, "f32");
    }
    // epilogue: bias and every activation, m = 2
    {
      const long long m = 2;
      const std::vector<float> x = activations(seed++, static_cast<size_t>(m * sp.cols));
      std::vector<float> bias = activations(seed++, static_cast<size_t>(sp.rows));
      sink.data(p + "_epi.x", x.data(), x.size() * 4, "f32");
      sink.data(p + "_epi.bias", bias.data(), bias.size() * 4, "f32");
      for (int a = 0; a < 5; ++a) {
        Out y(FT::kF32, m * sp.rows);
        const std::string c = p + "_epi" + std::to_string(a);
        sink.status(c, qc::qgemm_prepacked_epilogue_storage(
                           w, {x.data(), FT::kF32, m * sp.cols}, a % 2 ? bias.data() : nullptr,
                           y.view(), m, static_cast<qc::LinearActivation>(a)));
        put(sink, c + ".y", y);
      }
    }
    std::vector<float> x1 = activations(seed++, static_cast<size_t>(sp.cols));
    std::vector<float> y1(static_cast<size_t>(sp.rows), -1.0f);
    sink.data(p + "_gemv.x", x1.data(), x1.size() * 4, "f32");
    sink.status(p + "_gemv", qc::qgemv_prepacked(w, x1.data(), y1.data()));
    sink.data(p + "_gemv.y", y1.data(), y1.size() * 4, "f32");
  }

  // gate / up / SwiGLU and Q / K / V / RoPE over pairs of (B)-like tensors
  for (int affine = 0; affine < 2; ++affine) {
    const std::string p = affine ? "pa" : "ps";
    const long long group = affine ? 64 : 0;
    const qc::CanonicalQuantTensor tg = int8_tensor(100 + affine, 96, K, affine, group);
    const qc::CanonicalQuantTensor tu = int8_tensor(110 + affine, 96, K, affine, group);
    const qc::CanonicalQuantTensor tq = int8_tensor(120 + affine, 64, K, affine, group);
    const qc::CanonicalQuantTensor tk = int8_tensor(130 + affine, 32, K, affine, group);
    const qc::CanonicalQuantTensor tv = int8_tensor(140 + affine, 32, K, affine, group);
    const qc::CanonicalQuantTensor* all[] = {&tg, &tu, &tq, &tk, &tv};
    const char* names[] = {"g", "u", "q", "k", "v"};
    qc::CpuPackedWeights pw[5];
    for (int i = 0; i < 5; ++i) {
      sink.data(p + names[i] + ".codes", all[i]->data.data(), all[i]->data.size(), "i8");
      sink.data(p + names[i] + ".scales", all[i]->scales.data(), all[i]->scales.size() * 4, "f32");
      if (affine)
        sink.data(p + names[i] + ".zeros", all[i]->zero_points.data(),
                  all[i]->zero_points.size() * 4, "f32");
      sink.status(p + names[i] + "_prepare", pw[i].prepare(*all[i], qc::CpuPanelLayout::kAvx2Rows8));
    }
    for (long long m : {1LL, 3LL}) {
      const std::vector<float> x = activations(200 + affine + m, static_cast<size_t>(m * K));
      const std::string c = p + "_gu_m" + std::to_string(m);
      sink.data(c + ".x", x.data(), x.size() * 4, "f32");
      Out g(FT::kF32, m * 96), u(FT::kBF16, m * 96), s(FT::kF32, m * 96);
      sink.status(c, qc::qgemm_prepacked_gate_up_storage(pw[0], pw[1], {x.data(), FT::kF32, m * K},
                                                         g.view(), u.view(), m));
      put(sink, c + ".gate", g);
      put(sink, c + ".up", u);
      sink.status(c + "_swiglu", qc::qgemm_prepacked_swiglu_storage(
                                      pw[0], pw[1], {x.data(), FT::kF32, m * K}, s.view(), m));
      put(sink, c + "_swiglu.y", s);
      Out q(FT::kF32, m * 64), k(FT::kF16, m * 32), v(FT::kF32, m * 32);
      sink.status(c + "_qkv", qc::qgemm_prepacked_qkv_storage(pw[2], pw[3], pw[4],
                                                               {x.data(), FT::kF32, m * K},
                                                               q.view(), k.view(), v.view(), m));
      put(sink, c + "_qkv.q", q);
      put(sink, c + "_qkv.k", k);
      put(sink, c + "_qkv.v", v);
    }
    // RoPE: 4 query heads and 2 kv heads of 16, slot 1 of 3, position 2 of 4
    const std::vector<float> x = activations(300 + affine, static_cast<size_t>(K));
    std::vector<float> cs(4 * 8), sn(4 * 8);
    uint32_t s = 77u + affine;
    for (int i = 0; i < 32; ++i) {
      cs[i] = static_cast<float>(static_cast<int>(next(&s) % 201u) - 100) / 100.0f;
      sn[i] = static_cast<float>(static_cast<int>(next(&s) % 201u) - 100) / 100.0f;
    }
    sink.data(p + "_rope.x", x.data(), x.size() * 4, "f32");
    sink.data(p + "_rope.cos", cs.data(), cs.size() * 4, "f32");
    sink.data(p + "_rope.sin", sn.data(), sn.size() * 4, "f32");
    const FT ctypes[] = {FT::kF32, FT::kF16};
    for (FT ct : ctypes)
      for (int slot : {1, -1}) {
        Out q(FT::kF32, 64), kc(ct, 3 * 32), vc(ct, 3 * 32);
        const std::string c = p + "_rope_" + std::to_string(static_cast<int>(ct)) +
                              (slot < 0 ? "_noslot" : "_slot1");
        sink.status(c, qc::qgemv_prepacked_qkv_rope_kv_storage(
                           pw[2], pw[3], pw[4], {x.data(), FT::kF32, K}, cs.data(), sn.data(),
                           q.view(), kc.view(), vc.view(), 4, 2, 16, 3, 4, 2, slot));
        put(sink, c + ".q", q);
        put(sink, c + ".kc", kc);
        put(sink, c + ".vc", vc);
      }

    // invalid calls, each alone (statuses must equal the reference's)
    std::vector<float> y(96 * 4);
    std::vector<float> xx(4 * K);
    const qc::FloatStorageInput xi{xx.data(), FT::kF32, K};
    const qc::FloatStorageOutput yo{y.data(), FT::kF32, 96};
    qc::CpuPackedWeights empty;
    sink.status(p + "_bad_m0", qc::qgemm_prepacked_storage(pw[0], xi, yo, 0));
    sink.status(p + "_bad_xcount", qc::qgemm_prepacked_storage(pw[0], {xx.data(), FT::kF32, K - 1}, yo, 1));
    sink.status(p + "_bad_ycount", qc::qgemm_prepacked_storage(pw[0], xi, {y.data(), FT::kF32, 95}, 1));
    sink.status(p + "_bad_xtype", qc::qgemm_prepacked_storage(pw[0], {xx.data(), static_cast<FT>(7), K}, yo, 1));
    sink.status(p + "_bad_ytype", qc::qgemm_prepacked_storage(pw[0], xi, {y.data(), static_cast<FT>(5), 96}, 1));
    sink.status(p + "_bad_xnull", qc::qgemm_prepacked_storage(pw[0], {nullptr, FT::kF32, K}, yo, 1));
    sink.status(p + "_bad_ynull", qc::qgemm_prepacked_storage(pw[0], xi, {nullptr, FT::kF32, 96}, 1));
    sink.status(p + "_bad_act", qc::qgemm_prepacked_epilogue_storage(pw[0], xi, nullptr, yo, 1,
                                                                     static_cast<qc::LinearActivation>(9)));
    sink.status(p + "_bad_notready", qc::qgemm_prepacked_storage(empty, xi, yo, 1));
    sink.status(p + "_bad_gu_shape", qc::qgemm_prepacked_gate_up_storage(
                                         pw[0], pw[2], xi, yo, yo, 1));
    sink.status(p + "_bad_swiglu_null", qc::qgemm_prepacked_swiglu_storage(
                                            pw[0], pw[1], xi, {nullptr, FT::kF32, 96}, 1));
    sink.status(p + "_bad_qkv_count", qc::qgemm_prepacked_qkv_storage(
                                          pw[2], pw[3], pw[4], xi, {y.data(), FT::kF32, 64},
                                          {y.data(), FT::kF32, 31}, {y.data(), FT::kF32, 32}, 1));
    std::vector<float> kc(96), vc(96), q(64);
    auto rope = [&](long long hd, long long slots, long long maxp, int pos, int slot,
                    const float* cosp) {
      return qc::qgemv_prepacked_qkv_rope_kv_storage(
          pw[2], pw[3], pw[4], xi, cosp, sn.data(), {q.data(), FT::kF32, 64},
          {kc.data(), FT::kF32, 96}, {vc.data(), FT::kF32, 96}, 4, 2, hd, slots, maxp, pos, slot);
    };
    sink.status(p + "_bad_rope_hd", rope(15, 3, 4, 2, 1, cs.data()));
    sink.status(p + "_bad_rope_pos", rope(16, 3, 4, 4, 1, cs.data()));
    sink.status(p + "_bad_rope_slot", rope(16, 3, 4, 2, 3, cs.data()));
    sink.status(p + "_bad_rope_cache", rope(16, 2, 4, 2, 1, cs.data()));
    sink.status(p + "_bad_rope_null", rope(16, 3, 4, 2, 1, nullptr));
  }

  // weights prepared from GGUF bytes: no canonical layout
  {
    std::vector<uint8_t> blocks(8 * (K / 32) * 34, 0);
    for (size_t i = 0; i < blocks.size(); i += 34) blocks[i + 1] = 0x3c;   // d = 1.0
    qc::CpuPackedWeights g;
    sink.status("gguf_prepare", g.prepare(qc::QuantFormat::kQ8_0, blocks.data(), 8, K));
    std::vector<float> x(K, 0.5f), y(8);
    sink.status("gguf_storage", qc::qgemm_prepacked_storage(g, {x.data(), FT::kF32, K},
                                                            {y.data(), FT::kF32, 8}, 1));
    sink.status("gguf_gemv_prepacked", qc::qgemv_prepacked(g, x.data(), y.data()));
  }
}

}  // namespace storage_scenarios
