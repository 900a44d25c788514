// The int8 MFMA main loop shared by the W8A8 GEMM and the canonical int8
// row-plane projections: an output tile of TN rows of operand A ("W") by TM
// rows of operand B ("X"), both K-contiguous int8 matrices, accumulated
// exactly in int32 with v_mfma_i32_32x32x32_i8.  The caller owns the
// epilogue: it receives the wave's FN x FM grid of 32 x 32 accumulator
// tiles, in which lane l holds B row (lane & 31) of each tile and, in
// register e, A row 8 * (e >> 2) + 4 * (l >> 5) + (e & 3) -- four runs of
// four consecutive A rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qc_lds_dma.h"

namespace qc {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Output tile of workgroup `b` in an XCD-aware order.  Workgroups are handed
// to the 8 XCDs round-robin (b % 8), each with its own L2, so the tiles one
// XCD runs are made a contiguous range of a banded order (bands of kBandM
// m-tiles, n-tiles within a band): an XCD then reads few W and X panels.
constexpr int kXcds = 8;
constexpr int kBandM = 4;
__device__ __forceinline__ void tile_of(int b, int total, int tiles_n, int tiles_m, int& tn,
                                        int& tm) {
  const int q = total / kXcds, r = total % kXcds;
  const int xcd = b % kXcds, idx = b / kXcds;
  const int t = xcd * q + (xcd < r ? xcd : r) + idx;
  const int band = t / (tiles_n * kBandM);
  const int rem = t - band * tiles_n * kBandM;
  const int left = tiles_m - band * kBandM;
  const int gm = left < kBandM ? left : kBandM;
  tn = rem / gm;
  tm = band * kBandM + rem % gm;
}

__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// global_load_lds_dwordx4: every lane sends 16 bytes from its own global
// address to LDS byte lds + 16 * lane (`lds` is wave-uniform, passed in M0).
// The address-space cast only exists in the device pass.
__device__ __forceinline__ void load_lds16(const int8_t* g, int8_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
#endif
}

// The same with the non-temporal hint (nt), for bytes read once.
__device__ __forceinline__ void load_lds16_nt(const int8_t* g, int8_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 2);
#endif
}

// The same with 4 bytes per lane, to LDS byte lds + 4 * lane.
__device__ __forceinline__ void load_lds4(const void* g, int8_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
#endif
}

// Workgroup barrier for the direct-to-LDS pipeline.  __syncthreads() would
// make the compiler drain every outstanding global->LDS load (vmcnt(0)) and
// defeat the multi-stage prefetch; here the waits are explicit and the empty
// asm statements only stop the compiler moving memory accesses across.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The default per-quarter hook of Int8Ring::run_rows: nothing.  A hook
// whose kFresh is n > 0 consumes the sums of every n quarters (n dividing
// the quarters of a step): the MFMAs of each n-quarter run's first quarter
// then start from zero instead of accumulating, and the hook need not clear.
struct Int8NoStep {
  static constexpr int kFresh = 0;
  template <class Acc>
  __device__ void operator()(int, int, Acc&) const {}
};

// The default side data of Int8Ring::run_rows: none.  A side policy moves,
// per K step, kLoads global->LDS gathers of 4 bytes per lane and wave
// (issue(step, wave, stage_base): slots wave * kLoads + q, 256 bytes each,
// of that stage's side area) beside the operand tiles, on the same path, so
// the ring's waits and barriers cover them; read(step, stage_base) is called
// once per step, in order, before the hook of the step's quarter QPS - 2
// (its last quarter in the loop body, where the stage is still valid), to
// move what the hooks need into registers.  (A plain global load whose result is
// used while global->LDS loads are in flight makes the compiler wait for all
// of them: per-step data that way would drain the ring every step.)
struct Int8NoSide {
  static constexpr int kLoads = 0;
  __device__ void issue(int, int, int8_t*) const {}
  __device__ void read(int, const int8_t*) {}
};

// Operand B rows of a plain [M][K] matrix (rows past M clamped to M - 1).
struct Int8Rows {
  const int8_t* b;
  long long rows, k;
  __device__ const int8_t* operator()(long long r) const {
    return b + (r < rows ? r : rows - 1) * k;
  }
};

// Full-line ring (K % 32 == 0, both operands 16-byte aligned with rows K
// bytes apart).  Each K step covers KL bytes of every A and B row of the
// tile; with KL = 128 that is whole 128-byte cache lines, for which the
// global->LDS path delivers markedly more per CU than for half lines.
//
// LDS: an S-deep ring of stages; a stage holds A[TN][KL] then B[TM][KL],
// row-major, with the 16-byte chunk c of row r stored at position
// c ^ ((r >> 1) & (CPR - 1)).  A global_load_lds_dwordx4 moves 1 KB (RPL rows).
//
// MFMA: v_mfma_i32_32x32x32_i8 (one wavefront sustains close to the CU's
// int8 rate with it, unlike the 16x16x64 form).  A step is KL / 32 K
// quarters; the operand of quarter q for a 32-row fragment is, in lane l,
// row l&31, chunk 2q + (l>>5), the same lane->k map for A and B.  Those 64
// reads fall on all 16 four-bank slots 4 times each under the swizzle above.
//
// Schedule (wavefront-uniform, branch-free in the steady state):
//   prologue: issue the loads of steps 0..S-1 into stages 0..S-1;
//   step k, quarter q = 0..2: read the fragments of quarter q+1 while the
//     MFMAs of quarter q run;
//   quarter 3: wait for this wave's loads of step k+1, barrier (all waves'
//     loads are in and every wave has finished reading stage k), issue the
//     loads of step k+S into stage k (with S >= 3 only the first quarter of
//     them; the rest go out before the MFMAs of quarters 1..3 of step k+1),
//     read quarter 0 of step k+1, then the MFMAs of quarter 3.
// Past the last step the loads repeat the last step into stages that are
// never read again, which keeps every wait count a constant.  The last step
// runs separately and, when K is not a multiple of KL, skips the quarters
// past K (their loads read a clamped in-row address and are never used).
// Rows past N (A) or M (B) load a clamped in-range row; the epilogue must
// not store their products.
//
// NTB: every operand-B row is read by one workgroup only (one A tile along
// N), so its loads carry the non-temporal hint.
template <int TN, int TM, int S, int WGN, int WGM, int KL, bool NTB = false>
struct Int8Ring {
  static_assert(KL == 128 || KL == 64, "K step is a whole or a half cache line");
  static constexpr int QPS = KL / 32;                      // K quarters per step
  static constexpr int RPL = 1024 / KL;                    // rows per 1 KB load
  static constexpr int CPR = KL / 16;                      // 16-byte chunks per row
  static constexpr int NW = WGN * WGM;                     // WGN x WGM grid of wavefronts
  static constexpr int WN = TN / WGN, WM = TM / WGM;       // wave tile
  static constexpr int FN = WN / 32, FM = WM / 32;         // 32 x 32 tiles per wave
  static constexpr int GW = TN / RPL / NW;                 // 1 KB loads per wave per step (A)
  // B: GX per wave; when the B tile has fewer 1 KB blocks than there are
  // waves (BSPLIT), waves 0 .. TM / RPL - 1 load one each and the others none.
  static constexpr bool BSPLIT = TM / RPL < NW;
  static constexpr int GX = BSPLIT ? 1 : TM / RPL / NW;
  static constexpr int G = GW + GX;
  static constexpr int kStage = (TN + TM) * KL;
  static constexpr int kBytes = S * kStage;
  // LDS bytes with a side policy: its areas follow the S operand stages.
  template <class Side>
  static constexpr int kBytesWith = kBytes + S * NW * Side::kLoads * 256;
  static_assert(FN >= 1 && FM >= 1 && GW >= 1 && GX >= 1 && S >= 2, "tile shape");
  static_assert(!BSPLIT || TM % RPL == 0, "whole B blocks");
  static_assert(G * (S - 1) < 64, "vmcnt range");

  // Wave tile origin within the workgroup tile (A rows, B rows).
  __device__ static int wave_n(int wave) { return (wave / WGM) * WN; }
  __device__ static int wave_m(int wave) { return (wave % WGM) * WM; }

  // acc = sum over K of A[n0 + wave_n + ...] x B[m0 + wave_m + ...] for this
  // wave; `ring` is the workgroup's kBytes of LDS (1 KB aligned).
  __device__ static void run(const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M,
                             int N, int K, long long n0, long long m0, int8_t* ring,
                             v16i (&acc)[FN][FM]) {
    run_rows(A, Int8Rows{B, M, K}, N, K, n0, m0, ring, acc);
  }

  // The same with operand B row r at brow(r) (K bytes, 16-byte aligned, any
  // r the tile touches mapped to a readable row), and step(k, q, acc)
  // called once the MFMAs of quarter q (32 columns) of K step k are in acc,
  // quarters in order (it may fold and clear them: the next quarter
  // accumulates onto whatever it leaves).  With a side policy, `ring` holds
  // kBytesWith<Side> bytes.
  template <class BRow, class Step = Int8NoStep, class Side = Int8NoSide>
  __device__ static void run_rows(const int8_t* __restrict__ A, const BRow& brow, int N, int K,
                                  long long n0, long long m0, int8_t* ring, v16i (&acc)[FN][FM],
                                  Step step = Step(), Side* side = nullptr) {
    constexpr int XL = Side::kLoads;
    constexpr int GT = G + XL;                // loads per wave per step
    static_assert(GT * (S - 1) < 64, "vmcnt range");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    auto side_base = [&](int stage) { return ring + kBytes + stage * NW * XL * 256; };
    // (BSPLIT) this wave loads a B block: its loads per step are GT, else GT - 1
    const bool has_b = !BSPLIT || wave < TM / RPL;
    auto load_j = [&](int j) { return j < GW || has_b; };
    // wait until at most n steps' loads of this wave are in flight
    auto wait_steps = [&](auto n) {
      if constexpr (BSPLIT) {
        if (has_b) wait_vmcnt<GT * decltype(n)::value>();
        else wait_vmcnt<(GT - 1) * decltype(n)::value>();
      } else {
        wait_vmcnt<GT * decltype(n)::value>();
      }
    };

    // Load j of a wave covers operand rows r = RPL * (wave * GW + j) + lane / CPR
    // (A; likewise B with GX, which with BSPLIT is block `wave` for the waves
    // that load one), lane writing slot lane % CPR of its row.  Swizzle
    // key of row r: (r >> 1) & (CPR - 1).  128-byte lines: 4 * (the parity of
    // the load's 8-row block, wave * GW + j) + (lane >> 4) (j & 1 when GW is
    // even); 64-byte halves: (lane >> 3) & 3.
    const int8_t* src[G];
    int coff[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int par = (j < GW ? wave * GW + j : wave * GX + (j - GW)) & 1;
      coff[j] = KL == 128 ? ((lane & 7) ^ (4 * par + (lane >> 4))) * 16
                          : ((lane & 3) ^ ((lane >> 3) & 3)) * 16;
    }
#pragma unroll
    for (int j = 0; j < GW; ++j) {
      long long r = n0 + RPL * (wave * GW + j) + lane / CPR;
      r = r < N ? r : N - 1;
      src[j] = A + r * K;
    }
#pragma unroll
    for (int j = 0; j < GX; ++j) src[GW + j] = brow(m0 + RPL * (wave * GX + j) + lane / CPR);
    auto issue = [&](int step, int stage) {
      int8_t* base = ring + stage * kStage;
      const int k0 = step * KL;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        int off = k0 + coff[j];
        off = off < K - 16 ? off : K - 16;
        int8_t* dst = j < GW ? base + (wave * GW + j) * 1024
                             : base + TN * KL + (wave * GX + (j - GW)) * 1024;
        if (!load_j(j)) continue;
        if (NTB && j >= GW) load_lds16_nt(src[j] + off, dst);
        else load_lds16(src[j] + off, dst);
      }
      if constexpr (XL > 0) side->issue(step, wave, side_base(stage));
    };

    // Fragment offsets of quarter q within a 32-row block: row lane&31,
    // logical chunk 2q + (lane>>5), stored at that chunk ^ key(row).
    const int t = KL == 128 ? (lane >> 5) ^ ((lane >> 1) & 7) : (lane >> 5) ^ ((lane >> 1) & 3);
    int foff[QPS];
#pragma unroll
    for (int q = 0; q < QPS; ++q) foff[q] = (lane & 31) * KL + ((2 * q) ^ t) * 16;

#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    const int wn = wave_n(wave);
    const int wm = wave_m(wave);
    const int nq = K / 32;                    // K quarters in total
    const int nk = (nq + QPS - 1) / QPS;      // steps

    v4i fa[2][FN], fb[2][FM];
    auto read_frags = [&](int stage, int q, int slot) {
      const int8_t* sw = ring + stage * kStage + wn * KL + foff[q];
      const int8_t* sx = ring + stage * kStage + (TN + wm) * KL + foff[q];
#pragma unroll
      for (int i = 0; i < FN; ++i) fa[slot][i] = *reinterpret_cast<const v4i*>(sw + 32 * i * KL);
#pragma unroll
      for (int j = 0; j < FM; ++j) fb[slot][j] = *reinterpret_cast<const v4i*>(sx + 32 * j * KL);
    };
    // quarter qq of a step (a constant once the quarter loops are unrolled)
    constexpr int FRESH = Step::kFresh;
    static_assert(FRESH == 0 || QPS % FRESH == 0, "fresh runs within a step");
    auto mfmas = [&](int slot, int qq) {
      const bool fresh = FRESH > 0 && qq % (FRESH > 0 ? FRESH : 1) == 0;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = fresh ? __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[slot][i], fb[slot][j],
                                                                    v16i{}, 0, 0, 0)
                            : __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[slot][i], fb[slot][j],
                                                                    acc[i][j], 0, 0, 0);
    };

#pragma unroll
    for (int st = 0; st < S; ++st) issue(st < nk ? st : nk - 1, st);
    wait_steps(std::integral_constant<int, S - 1>());
    ring_barrier();
    read_frags(0, 0, 0);
    // With three or more stages the loads of a step are spread over the
    // quarters of the next one (part 0 after the barrier, part q before
    // quarter q's MFMAs) instead of being queued by all waves at once: they
    // are needed only S - 2 steps later.  With two stages they are needed at
    // the end of the next step and go out together.
    constexpr int SPREAD = S >= 3 ? QPS : 1;
    int stage = 0;
    int pstep = 0, pstage = 0;                // the step being loaded and its stage
    auto issue_part = [&](int part) {
      int8_t* base = ring + pstage * kStage;
      const int k0 = pstep * KL;
#pragma unroll
      for (int j = part * G / SPREAD; j < (part + 1) * G / SPREAD; ++j) {
        int off = k0 + coff[j];
        off = off < K - 16 ? off : K - 16;
        int8_t* dst = j < GW ? base + (wave * GW + j) * 1024
                             : base + TN * KL + (wave * GX + (j - GW)) * 1024;
        if (!load_j(j)) continue;
        if (NTB && j >= GW) load_lds16_nt(src[j] + off, dst);
        else load_lds16(src[j] + off, dst);
      }
      if constexpr (XL > 0)
        if (part == 0) side->issue(pstep, wave, side_base(pstage));
    };
    // Side data is read with the fragments of the step's last in-loop quarter
    // (the stage is refilled after the barrier).
    static_assert(XL == 0 || QPS > 1, "side data read within the quarter loop");
    for (int k = 0; k + 1 < nk; ++k) {
#pragma unroll
      for (int q = 1; q < QPS; ++q) {
        if (q < SPREAD && k > 0) issue_part(q);
        read_frags(stage, q, q & 1);
        if constexpr (XL > 0)
          if (q == QPS - 1) side->read(k, side_base(stage));
        mfmas((q - 1) & 1, q - 1);
        step(k, q - 1, acc);
      }
      // Loads issued: steps up to k+S-1, all parts; step k+1 must be in.
      wait_steps(std::integral_constant<int, S - 2>());
      wait_lgkmcnt0();
      ring_barrier();
      pstep = k + S < nk ? k + S : nk - 1;
      pstage = stage;
      issue_part(0);
      stage = stage + 1 < S ? stage + 1 : 0;
      read_frags(stage, 0, 0);
      mfmas((QPS - 1) & 1, QPS - 1);
      step(k, QPS - 1, acc);
    }
    {
      if constexpr (XL > 0) side->read(nk - 1, side_base(stage));
      const int qn = nq - QPS * (nk - 1);    // 1..QPS quarters in the last step
#pragma unroll
      for (int q = 1; q < QPS; ++q) {
        if (q < qn) read_frags(stage, q, q & 1);
        if (q - 1 < qn) {
          mfmas((q - 1) & 1, q - 1);
          step(nk - 1, q - 1, acc);
        }
      }
      if (QPS - 1 < qn) {
        mfmas((QPS - 1) & 1, QPS - 1);
        step(nk - 1, QPS - 1, acc);
      }
    }
    // No global->LDS load may still be in flight when the workgroup's LDS is
    // released.
    wait_vmcnt<0>();
  }
};

}  // namespace qc
