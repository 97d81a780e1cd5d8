// Flash-attention forward (non-causal) for gfx950: O = softmax(Q K^T * sm_scale) V
// per (batch, query head), with grouped K/V heads (query head h reads K/V head
// h * HK / HQ).  Head dim 128 or 64, FP16 or BF16 in and out, fp32 softmax
// and accumulation.  extern "C" entry: g9_fmha_fwd (include/gfx950_fmha.h).
//
// One workgroup owns 256 query rows of one (batch, head) and walks all keys in
// tiles of 8192 / D keys (64 at head dim 128, 128 at 64).  Its 8 waves (2 per
// SIMD) own 32 query rows each, so every row-wise reduction stays inside a
// wave.  Per key tile a wave runs
//   S^T = K . Q^T    16 MFMAs 32x32x16 (32-key blocks x D/16 steps of 16 d);
//                    K fragments from LDS, Q fragments in registers;
//   online softmax   running max m and (lane-partial) sum l in log2 units;
//   O^T += V^T . P^T 16 MFMAs (D/32 blocks of 32 d x steps of 16 keys);
//                    P^T straight from the S^T registers, V^T through LDS
//                    transpose reads.
// The scores are computed transposed (the keys are the MFMA's rows): lane l
// then holds 16 keys of query l % 32 per 32-key block, so the row max and
// the row sum of a query are in-lane reductions plus one exchange with lane
// l ^ 32, the accumulator rescale is one per-lane factor, and the score
// registers are already the B operand of the PV MFMA once its 16-key steps use
// the key order the score layout gives each lane half: step t, lane half h,
// slot u covers key 16t + 8(u / 4) + 4h + (u % 4).  V is read in that key order
// with ds_read_b64_tr_b16, which within each 16-lane group gives lane 4a + b
// element b of the 8-byte rows addressed by lanes a, a + 4, a + 8, a + 12
// (measured on gfx950): 4 keys of one head-dim column per read.
//
// The loop is software pipelined over four clusters with the two waves of a
// SIMD one cluster apart (see Pipe below).
#include <stdint.h>

#include "../../include/gfx950_fmha.h"
#include "g9_common.hpp"

namespace g9 {
namespace fa {

// Optional phase stamps (build with -DG9_TIMING; read by profiling.py through
// g9_fmha_timing_read): thread 0 of each workgroup records s_memtime (shader
// clock) and s_memrealtime (100 MHz) at kernel entry, loop start, loop end and
// kernel end, for the first kTimingWorkgroups workgroups (by block index).
// Each stamp waits only for its own scalar reads.  Nothing in the regular
// build.
#ifdef G9_TIMING
constexpr int kTimingWorkgroups = 16384;
__device__ unsigned long long g9_fmha_timing_buf[kTimingWorkgroups * 8];
G9_DEV void stamp(int slot) {
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t = __builtin_amdgcn_s_memtime();
  const unsigned long long r = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_s_waitcnt((63 & 15) | (7 << 4) | (0 << 8) | ((63 >> 4) << 14));  // lgkmcnt(0) only
  if (threadIdx.x == 0 && blockIdx.x < kTimingWorkgroups) {
    g9_fmha_timing_buf[blockIdx.x * 8 + slot * 2] = t;
    g9_fmha_timing_buf[blockIdx.x * 8 + slot * 2 + 1] = r;
  }
  __builtin_amdgcn_sched_barrier(0);
}
#else
G9_DEV void stamp(int) {}
#endif

constexpr int kBlockM = 256;                // query rows per workgroup
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazyThreshold = 8.f;       // log2 units: p < 256 between rescales

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

struct FaParams {
  const char* q;
  const char* k;
  const char* v;
  char* o;
  float* lse;                        // [B][HQ][S] fp32, or null
  long long q_b, q_h, k_b, k_h, v_b, v_h, o_b, o_h;  // batch / head strides, bytes
  u32 ldq, ldk, ldv, ldo;            // sequence strides, bytes
  int B, HQ, HK, S;
  int mblocks;                       // ceil(S / 256)
  int num_xcds;
  float scale_log2;                  // sm_scale * log2(e)
  int scale_on_q;                    // fold scale_log2 into Q (rounded to 16 bit) before the loop
};

// MFMA 32x32x16 on 16-bit operands given as raw registers.
template <bool BF16>
G9_DEV f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// Two fp32 values -> one register of two 16-bit values (round to nearest even).
template <bool BF16>
G9_DEV u32 pack2(float x, float y) {
  if constexpr (BF16) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(u32, __builtin_convertvector((f32x2){x, y}, b2));
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(u32, __builtin_convertvector((f32x2){x, y}, h2));
  }
}

// Two 16-bit values of one register -> fp32.
template <bool BF16>
G9_DEV f32x2 unpack2(u32 w) {
  if constexpr (BF16) {
    return f32x2{__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_convertvector(__builtin_bit_cast(h2, w), f32x2);
  }
}

// Value of lane l ^ 32 combined with this lane's by a symmetric op.
template <class F>
G9_DEV float xhalf(float x, F op) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return op(__int_as_float(r[0]), __int_as_float(r[1]));
}

// LDS-DMA of 16 bytes per lane (lane i writes lds + 16 i, reading global
// voff + soff) issued as inline assembly, so the compiler does not track it:
// it adds no wait for these DMAs before LDS reads (it cannot tell the read
// addresses from the DMA targets apart and would wait for every DMA in
// flight).  The caller orders them with explicit vmcnt waits and barriers.
// The LDS address goes in through an M0 operand, so the compiler writes M0
// itself and knows what it holds.
G9_DEV void dma16_untracked(rsrc_t r, u32 lds, u32 voff, u32 soff) {
  asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" : : "{m0}"(lds), "v"(voff), "s"(r), "s"(soff) : "memory");
}

// Pins a value to this point of the program: the compiler can neither move
// its computation past the statement nor sink it toward its uses.
G9_DEV void pin(float& x) { asm volatile("" : "+v"(x)); }
G9_DEV void pin(u32& x) { asm volatile("" : "+v"(x)); }
template <class V>
G9_DEV void pin_vec(V& v) {
#pragma unroll
  for (int i = 0; i < (int)(sizeof(V) / 4); ++i) {
    float x = v[i];
    pin(x);
    v[i] = x;
  }
}

G9_DEV u32x2 tr_read(u32 addr) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((G9_LDS s16x4*)(uintptr_t)addr);
  return __builtin_bit_cast(u32x2, r);
}

// ---------------------------------------------------------------------------
// Pipelined form.  Each wave's loop over key tiles j is cut into four
// clusters, each closed by a workgroup barrier:
//   D1(j)  QK MFMAs of tile j+1 (K_{j+1} from registers) and, in their issue
//          shadow, the second half of tile j's softmax (the remaining
//          exponentials, P_j to 16 bit, the row sum) and, with the eager
//          rescale, half of O's rescale for tile j;
//   M1(j)  LDS reads of V_j; DMA of K_{j+3}; tile j+1's row max, new running
//          max and rescale factor (a dependent chain: it would stall MFMA
//          issue in a dot cluster, here it fills the idle VALU);
//   D2(j)  PV MFMAs of tile j and, in their shadow, most of tile j+1's
//          exponentials;
//   M2(j)  LDS reads of K_{j+2}; DMA of V_{j+2}; rescale of l and (the rest of) O.
// Waves 4-7 run one cluster behind waves 0-3, so on every SIMD one wave is in
// a dot cluster (MFMA + VALU) while the other is in a memory cluster: the
// matrix pipe, the VALU and the LDS / memory pipe are busy at the same time.
// Memory clusters run at wave priority 1, dot clusters at 0, so the memory
// wave's reads, DMAs and rescale win issue arbitration (measured: 2.5% fewer
// loop cycles with the lazy rescale; the priority of M2 is what matters).
// K and V tiles are double buffered in LDS (tile t in buffer t & 1); each DMA
// is waited for (by its own wave, then a barrier) one cluster before the tile
// is read, which gives it about one and a half loop iterations to land.
//
// LDS tiles are stored column-major in 16-byte chunks: chunk c (head-dim
// values 8c..8c+7) of all kBN rows is contiguous (one DMA per 64 rows: lane i
// fetches row i), chunk columns kPitchK / kPitchV bytes apart.  Every LDS read
// address is then one per-lane base register plus an immediate: K reads
// (row = lane % 32 (+32), chunk 2s + lane / 32) cover 256 contiguous bytes per
// 16 lanes; a V transpose read of 16 lanes covers 4 rows of two adjacent
// chunks, 64 bytes each, which the 64-byte pad of kPitchV puts on distinct
// banks.
// ---------------------------------------------------------------------------

#ifndef G9_FMHA_VN1
#define G9_FMHA_VN1 4  // VALU instructions after each QK MFMA of D1
#endif
#ifndef G9_FMHA_VN1_EAGER
#define G9_FMHA_VN1_EAGER 6  // the same with the eager rescale's share of O in D1
#endif
#ifndef G9_FMHA_VN2
#define G9_FMHA_VN2 4  // VALU instructions after each PV MFMA of D2
#endif
#ifndef G9_FMHA_VEC1_EXPS
#define G9_FMHA_VEC1_EXPS 22  // exponentials of a tile done in D2 (of 32 per lane); the rest in D1
#endif

#ifndef G9_FMHA_VN1_64
#define G9_FMHA_VN1_64 8  // head dim 64 (128-key tiles): VALU after each QK MFMA of D1
#endif
#ifndef G9_FMHA_VN2_64
#define G9_FMHA_VN2_64 8  // head dim 64: VALU after each PV MFMA of D2
#endif
#ifndef G9_FMHA_VEC1_EXPS_64
#define G9_FMHA_VEC1_EXPS_64 44  // head dim 64: exponentials of a tile (of 64 per lane) done in D2
#endif

// Sum of a 16-entry table (compile time).
constexpr int sum16(const int (&a)[16]) {
  int t = 0;
  for (int i = 0; i < 16; ++i) t += a[i];
  return t;
}

// SOQ: the scale is folded into Q, so the scores already are in log2 units
// and the exponent argument is a 2-source subtract instead of a 3-source fma
// (fewer register-file reads beside the other wave's LDS returns).
//
// Key tiles are kBN = 8192 / HD keys: 64 at head dim 128, 128 at head dim 64,
// so a dot cluster holds 16 MFMAs either way and the two head dims share the
// per-cluster costs (barriers, the row-max chain, waits) over the same MFMA
// work.  A tile's scores are kNB blocks of 32 keys (Sc).
template <bool BF16, bool LAZY, bool SOQ, int HD>
struct Pipe {
  static_assert(HD == 64 || HD == 128, "head dim 64 or 128");
  static constexpr int kBN = 8192 / HD;        // keys per tile
  static constexpr int kNB = kBN / 32;         // 32-key score blocks per tile
  static constexpr int kKS = kBN / 16;         // PV steps of 16 keys
  static constexpr int kNS = HD / 16;          // QK steps of 16 head-dim values
  static constexpr int kND = HD / 32;          // PV blocks of 32 head-dim values
  static constexpr int kNC = HD / 8;           // 16-byte chunk columns per row
  static constexpr int kNF = kNS * kNB;        // K (or V) fragments per tile = MFMAs per dot cluster
  static constexpr int kRH = kBN / 64;         // 64-row halves of a chunk column (one DMA each)
  static constexpr int kDW = kNC * kRH / kWaves;  // DMAs per wave per operand and tile
  static constexpr int kPitchK = kBN * 16;     // bytes between K chunk columns
  static constexpr int kPitchV = kBN * 16 + 64;  // bytes between V chunk columns (pad: distinct banks)
  static constexpr int kTileK = kNC * kPitchK;  // one K tile in LDS
  static constexpr int kTileV = kNC * kPitchV;  // one V tile in LDS
  static constexpr int kLdsV = 2 * kTileK;     // V buffers after the two K buffers
  static constexpr int kLdsBytes = 2 * kTileK + 2 * kTileV;
  static constexpr int kE1 = HD == 128 ? G9_FMHA_VEC1_EXPS : G9_FMHA_VEC1_EXPS_64;
  static constexpr int kVN1 = HD == 128 ? G9_FMHA_VN1 : G9_FMHA_VN1_64;
  static constexpr int kVN2 = HD == 128 ? G9_FMHA_VN2 : G9_FMHA_VN2_64;
  static_assert(kNF == 16 && kKS * kND == 16, "16 MFMAs per dot cluster");
  struct Sc {
    f32x16 b[kNB];
  };
  const FaParams& p;
  int nt, nte, nfull, wave;  // tiles, tiles rounded up to even, whole tiles, wave index
  u32 lds0;
  rsrc_t rk, rv;
  u32 voffk, voffv;  // lane's row offset in global K / V
  u32 ak, av;        // lane's LDS read base for K / V
  float sc;
  u32x4 qf[kNS];
  u32x4 kv[kNF];  // K_t (kv[kNB s + blk]: step s of 16 head-dim values, key block blk) or V_t (kv[kND t + d])
  f32x16 o[kND];  // O^T, head-dim block d
  float m, l, alpha;

  G9_DEV explicit Pipe(const FaParams& pp) : p(pp) {}

  // DMA q = kDW w + i of wave w covers chunk column q / kRH, rows 64 (q % kRH)
  // .. +63 of a tile: lane i fetches row 64 (q % kRH) + i.
  G9_DEV void dma_k(int tile, int buf) {
#pragma unroll
    for (int i = 0; i < kDW; ++i) {
      const int q = kDW * wave + i, c = q / kRH, r = q % kRH;
      dma16_untracked(rk, lds0 + buf * kTileK + c * kPitchK + r * 1024, voffk,
                      ((u32)tile * kBN + 64 * r) * p.ldk + c * 16);
    }
  }
  G9_DEV void dma_v(int tile, int buf) {
#pragma unroll
    for (int i = 0; i < kDW; ++i) {
      const int q = kDW * wave + i, c = q / kRH, r = q % kRH;
      dma16_untracked(rv, lds0 + kLdsV + buf * kTileV + c * kPitchV + r * 1024, voffv,
                      ((u32)tile * kBN + 64 * r) * p.ldv + c * 16);
    }
  }
  template <int BUF>
  G9_DEV void read_k() {
#pragma unroll
    for (int s = 0; s < kNS; ++s)
#pragma unroll
      for (int blk = 0; blk < kNB; ++blk)
        kv[kNB * s + blk] = *(const G9_LDS u32x4*)(uintptr_t)(ak + BUF * kTileK + 2 * s * kPitchK + blk * 512);
  }
  template <int BUF>
  G9_DEV void read_v() {
#pragma unroll
    for (int t = 0; t < kKS; ++t)
#pragma unroll
      for (int d = 0; d < kND; ++d) {
        const u32 a = av + BUF * kTileV + 4 * d * kPitchV + 256 * t;
        const u32x2 lo = tr_read(a);
        const u32x2 hi = tr_read(a + 128);
        kv[kND * t + d] = u32x4{lo.x, lo.y, hi.x, hi.y};
      }
  }
  // S^T of the tile in kv: kNB 32-key blocks.
  G9_DEV void qk(Sc& S) {
#pragma unroll
    for (int blk = 0; blk < kNB; ++blk) S.b[blk] = mfma<BF16>(kv[blk], qf[0], f32x16{});
#pragma unroll
    for (int s = 1; s < kNS; ++s)
#pragma unroll
      for (int blk = 0; blk < kNB; ++blk) S.b[blk] = mfma<BF16>(kv[kNB * s + blk], qf[s], S.b[blk]);
  }
  // O^T += V^T P^T; P in 16 bit as vec2 left it in S.
  G9_DEV void pv(const Sc& S) {
#pragma unroll
    for (int t = 0; t < kKS; ++t) {
      const f32x16& sv = S.b[t / 2];
      const u32x4 pt = t & 1 ? __builtin_bit_cast(u32x4, __builtin_shufflevector(sv, sv, 8, 9, 10, 11))
                             : __builtin_bit_cast(u32x4, __builtin_shufflevector(sv, sv, 0, 1, 2, 3));
#pragma unroll
      for (int d = 0; d < kND; ++d) o[d] = mfma<BF16>(kv[kND * t + d], pt, o[d]);
    }
  }
  // p = 2^(x * sc - m) for score register i (0 .. 16 kNB - 1) of a lane:
  // block i / 16, register i % 16.
  G9_DEV void expo(Sc& S, int i) const {
    f32x16& v = S.b[i / 16];
    v[i % 16] = __builtin_amdgcn_exp2f(SOQ ? v[i % 16] - m : __builtin_fmaf(v[i % 16], sc, -m));
  }
  // Keys past the sequence end (the phantom tile, or the second half of a
  // 128-key tile when S is an odd multiple of 64) score -inf: their K rows
  // were read as zeros.  `valid` = keys of the tile before the end (a
  // multiple of 64, <= 0 for the phantom).
  G9_DEV void mask(Sc& S, int valid) const {
    const int from = kBN == 64 || valid <= 0 ? 0 : kNB / 2;  // whole-tile stores, no selects
#pragma unroll
    for (int blk = 0; blk < kNB; ++blk)
      if (blk >= from) S.b[blk] = f32x16{} - __builtin_inff();
  }

  // Start of a tile's softmax: row max, running max and alpha (a dependent
  // chain ending in a cross-lane exchange; run in a memory cluster, where the
  // VALU is otherwise idle, so the MFMA shadows keep only independent work).
  // One max3 chain per 8-register half block, then a tree over the chains.
  G9_DEV void vec0(Sc& S) {
    float c[2 * kNB];
#pragma unroll
    for (int h = 0; h < 2 * kNB; ++h) {
      const f32x16& v = S.b[h / 2];
      const int o8 = 8 * (h & 1);
      c[h] = __builtin_fmaxf(__builtin_fmaxf(v[o8], v[o8 + 1]), v[o8 + 2]);
    }
#pragma unroll
    for (int i = 3; i < 8; i += 2) {
      const int i1 = i + 1 < 8 ? i + 1 : i;
#pragma unroll
      for (int h = 0; h < 2 * kNB; ++h) {
        const f32x16& v = S.b[h / 2];
        const int o8 = 8 * (h & 1);
        c[h] = __builtin_fmaxf(__builtin_fmaxf(c[h], v[o8 + i]), v[o8 + i1]);
      }
    }
#pragma unroll
    for (int w = 2 * kNB; w > 1; w /= 2)
#pragma unroll
      for (int h = 0; h < w / 2; ++h) c[h] = __builtin_fmaxf(c[2 * h], c[2 * h + 1]);
    float mx = c[0];
    mx = xhalf(mx, [](float x, float y) { return __builtin_fmaxf(x, y); });
    const float mt = SOQ ? mx : mx * sc;
    const float m_new = LAZY ? (mt - m > kLazyThreshold ? mt : m) : __builtin_fmaxf(m, mt);
    alpha = __builtin_amdgcn_exp2f(m - m_new);
    m = m_new;
  }
  // First kE1 exponentials of a tile (in place).
  G9_DEV void vec1(Sc& S) {
#pragma unroll
    for (int i = 0; i < kE1; ++i) expo(S, i);
  }
  // Second half: the remaining exponentials, l += row sum (fp32, before
  // rounding), P to 16 bit.  The 16-bit pairs of PV step t are written over
  // the first four registers of their eight scores (registers 8(t % 2) .. +3
  // of block t / 2), so P needs no registers of its own.  (The row sum uses
  // plain adds: v_dot2c on the packed values would take half the
  // instructions but does not issue beside an MFMA -- measured: two per MFMA
  // stretch its 32-cycle interval to 53.)
  G9_DEV void vec2(Sc& S) {
#pragma unroll
    for (int i = kE1; i < 16 * kNB; ++i) expo(S, i);
    float r[2 * kNB];
#pragma unroll
    for (int h = 0; h < 2 * kNB; ++h) {
      const f32x16& v = S.b[h / 2];
      const int o8 = 8 * (h & 1);
      r[h] = v[o8] + v[o8 + 1];
    }
#pragma unroll
    for (int i = 2; i < 8; ++i)
#pragma unroll
      for (int h = 0; h < 2 * kNB; ++h) r[h] += S.b[h / 2][8 * (h & 1) + i];
#pragma unroll
    for (int w = 2 * kNB; w > 1; w /= 2)
#pragma unroll
      for (int h = 0; h < w / 2; ++h) r[h] = r[2 * h] + r[2 * h + 1];
    l += r[0];
#pragma unroll
    for (int t = 0; t < kKS; ++t) {
      f32x16& sv = S.b[t / 2];
      const int r0 = 8 * (t & 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[r0 + e] = __uint_as_float(pack2<BF16>(sv[r0 + 2 * e], sv[r0 + 2 * e + 1]));
    }
  }
  // Pins the 16-bit P pairs and l (vec2's results).
  G9_DEV void pin_p(Sc& S) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int blk = 0; blk < kNB; ++blk) {
        float a = S.b[blk][e], b = S.b[blk][8 + e];
        pin(a), pin(b);
        S.b[blk][e] = a, S.b[blk][8 + e] = b;
      }
    pin(l);
  }
  G9_DEV void pin_sc(Sc& S) {
#pragma unroll
    for (int blk = 0; blk < kNB; ++blk) pin_vec(S.b[blk]);
  }
  // The eager rescale (every tile) at head dim 128 splits O: the first kSplit
  // head-dim blocks are rescaled in the next dot cluster, as VALU work beside
  // the QK MFMAs (rescale_early), the rest here (measured: 7.5% fewer loop
  // cycles than all of it here; at head dim 64, whose dot clusters have half
  // the MFMAs, 1.5% more).  The lazy rescale is rare and stays here whole.
  // Both skip the multiplies here when no row of the wave moved its max
  // (alpha is then exactly 1, so the skip changes no bit; eager rescale: 1.8%
  // fewer loop cycles at S=8192, where later tiles rarely move a row's max).
  static constexpr int kSplit = LAZY || HD != 128 ? 0 : kND / 2;
  G9_DEV void rescale() {
    l *= alpha;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int d = kSplit; d < kND; ++d) o[d] *= alpha;
    }
  }
  G9_DEV void rescale_early() {
#pragma unroll
    for (int d = 0; d < kSplit; ++d) o[d] *= alpha;
  }

  // Interleave of a dot cluster (kNF MFMAs): MFMA i followed by VN VALU
  // instructions and exps_in_slot() exponentials.  An MFMA 32x32x16 takes 32
  // cycles; about six plain VALU instructions or two to three exponentials
  // issue beside it without delaying the next one (measured).  Exponentials
  // are not in the VALU class of sched_group_barrier; left to the scheduler
  // they bunch up (5-8 in one MFMA slot, none in the next ten), so each slot
  // gets its own count.  D1 (W = 1) finishes tile j's exponentials, which its
  // row sums and 16-bit conversions consume later in the same cluster, so
  // they go early; D2 (W = 2) starts tile j+1's, which nothing in D2 reads,
  // so they are spread out.  The counts were chosen by measurement (loop
  // cycles at B=32 S=8192 bf16: head dim 128 v4 -3.4%, v3 +-0; head dim 64
  // -3.8% and -3.0% against the spread the scheduler picks; the sum over a
  // cluster is the exponentials it holds: 10 and 22 of 32 at head dim 128,
  // 20 and 44 of 64 at 64).
  static constexpr int kEp1[16] = {1, 1, 1, 1, 1, 1, 1, 1, 1, 1};  // D1, lazy rescale
  static constexpr int kEp1e[16] = {4, 3, 3};  // D1 beside the eager rescale's 6 VALU per slot
  static constexpr int kEp2[16] = {1, 1, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2};
  static constexpr int kEp1_64[16] = {1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2};
  static constexpr int kEp2_64[16] = {2, 3, 3, 3, 3, 3, 3, 3, 3, 3, 3, 3, 3, 3, 3};
  template <int W, int I>
  G9_DEV static constexpr int exps_in_slot() {
    if constexpr (HD == 128)
      return W == 1 ? (LAZY ? kEp1[I] : kEp1e[I]) : kEp2[I];
    else
      return W == 1 ? kEp1_64[I] : kEp2_64[I];
  }
  static_assert(HD != 128 || sum16(kEp1) == 32 - kE1, "D1 exponentials per slot: re-chosen with the D1/D2 split");
  static_assert(HD != 128 || sum16(kEp1e) == 32 - kE1, "D1 exponentials per slot: re-chosen with the D1/D2 split");
  static_assert(HD != 128 || sum16(kEp2) == kE1, "D2 exponentials per slot: re-chosen with the D1/D2 split");
  static_assert(HD == 128 || sum16(kEp1_64) == 64 - kE1, "D1 exponentials per slot: re-chosen with the D1/D2 split");
  static_assert(HD == 128 || sum16(kEp2_64) == kE1, "D2 exponentials per slot: re-chosen with the D1/D2 split");
  template <int VN, int W, int I = 0>
  G9_DEV static void interleave() {
    if constexpr (I < kNF) {
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
      __builtin_amdgcn_sched_group_barrier(SG_VALU, VN, 0);
      constexpr int e = exps_in_slot<W, I>();
      if constexpr (e > 0) __builtin_amdgcn_sched_group_barrier(SG_TRANS, e, 0);
      interleave<VN, W, I + 1>();
    }
  }

  // One loop iteration; PAR = j & 1 fixes the LDS buffers; c holds tile j's
  // scores after vec1, n receives tile j+1's; NEXT: tile j+1 exists.  The
  // loop runs over an even number of tiles nte: when nt is odd the last tile
  // is a phantom past the end of the sequence (its DMAs read zeros from the
  // buffer range check) whose scores are set to -inf, so it adds nothing.
  // Registers are written unconditionally (a read past the last tile reads a
  // stale but in-bounds buffer), so no value has to survive a skipped branch.
  template <int PAR, bool NEXT>
  G9_DEV void step(int j, Sc& c, Sc& n) {
    // D1(j)
    __builtin_amdgcn_s_setprio(0);
    if constexpr (NEXT) {
      qk(n);
      vec2(c);
      rescale_early();
      interleave<(kSplit ? G9_FMHA_VN1_EAGER : kVN1), 1>();
      pin_sc(n);
    } else {
      vec2(c);
      rescale_early();
    }
#pragma unroll
    for (int d = 0; d < kSplit; ++d) pin_vec(o[d]);
    pin_p(c);
    barrier();
    // M1(j): V_j was waited for at the end of M2(j-1) (or the prologue).
    __builtin_amdgcn_s_setprio(1);
    read_v<PAR>();
    if (j + 2 < nte) waitcnt<kDW, 15>();  // K_{j+2} landed (V_{j+1} may be in flight)
    if (j + 3 < nte) dma_k(j + 3, PAR ^ 1);
    if constexpr (NEXT) {
      if (j + 1 >= nfull) {  // past the end (a branch, not selects in every step)
        asm volatile("");
        mask(n, p.S - (j + 1) * kBN);
      }
      vec0(n);
      pin(m);
      pin(alpha);
    }
    waitcnt<63, 0>();
    barrier();
    // D2(j)
    __builtin_amdgcn_s_setprio(0);
    if constexpr (NEXT) {
      pv(c);
      vec1(n);
      interleave<kVN2, 2>();
      pin_sc(n);
    } else {
      pv(c);
    }
#pragma unroll
    for (int d = 0; d < kND; ++d) pin_vec(o[d]);
    barrier();
    // M2(j)
    __builtin_amdgcn_s_setprio(1);
    if constexpr (NEXT) {
      read_k<PAR>();
      if (j + 3 < nte)
        waitcnt<kDW, 15>();  // V_{j+1} landed (K_{j+3} may be in flight)
      else
        waitcnt<0, 15>();
      rescale();
    }
    if (j + 2 < nte) dma_v(j + 2, PAR);
    waitcnt<63, 0>();
    barrier();
  }
};

// smem: PipeT::kLdsBytes of LDS, 1024-byte aligned, declared by the kernel
// (one array for both scale placements a kernel instantiates).
template <bool BF16, bool LAZY, bool SOQ, int HD>
G9_DEV void fmha_fwd(const FaParams& p, char* smem) {
  using PipeT = Pipe<BF16, LAZY, SOQ, HD>;
  stamp(0);
  const int total = p.B * p.HQ * p.mblocks;
  int pid, unused;
  tile_coords(blockIdx.x, total, total, 1, p.num_xcds, 1, pid, unused);
  const int bh = pid / p.mblocks, mb = pid - bh * p.mblocks;
  const int b = bh / p.HQ, hq = bh - b * p.HQ;
  const int hk = hq * p.HK / p.HQ;
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = lane >> 5;

  PipeT P(p);
  P.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  P.nt = (p.S + PipeT::kBN - 1) / PipeT::kBN;
  P.nte = (P.nt + 1) & ~1;
  P.nfull = p.S / PipeT::kBN;
  P.lds0 = (u32)(uintptr_t)to_lds(smem);
  const int nte = P.nte, wave = P.wave;
  const char* qb = p.q + b * p.q_b + hq * p.q_h;
  const rsrc_t rq = make_rsrc(qb, (u32)p.S * p.ldq);
  P.rk = make_rsrc(p.k + b * p.k_b + hk * p.k_h, (u32)p.S * p.ldk);
  P.rv = make_rsrc(p.v + b * p.v_b + hk * p.v_h, (u32)p.S * p.ldv);

  const int qrow = mb * kBlockM + wave * 32 + (lane & 31);
#pragma unroll
  for (int s = 0; s < PipeT::kNS; ++s)
    P.qf[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (u32)qrow * p.ldq + (16 * s + 8 * h) * 2, 0, 0));
  P.voffk = (u32)lane * p.ldk;
  P.voffv = (u32)lane * p.ldv;
  P.ak = P.lds0 + h * PipeT::kPitchK + (lane & 31) * 16;
  {
    const int G = lane >> 4, jj = lane & 15;
    P.av = P.lds0 + PipeT::kLdsV + (2 * (G & 1) + ((jj & 3) >> 1)) * PipeT::kPitchV + (4 * (G >> 1) + (jj >> 2)) * 16 +
           8 * (jj & 1);
  }
  // Prologue: K_0, V_0, K_1 in; S_0 and its first softmax half; K_2 and V_1
  // requested (in that order: the loop expects K_{j+2} before V_{j+1}); K_1
  // in registers.
  P.dma_k(0, 0);
  P.dma_v(0, 0);
  P.dma_k(1, 1);
  P.sc = p.scale_log2;
  if constexpr (SOQ) {
#pragma unroll
    for (int s = 0; s < PipeT::kNS; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f32x2 x = unpack2<BF16>(P.qf[s][e]);
        P.qf[s][e] = pack2<BF16>(x.x * P.sc, x.y * P.sc);
      }
    P.sc = 1.f;
  }
#pragma unroll
  for (int d = 0; d < PipeT::kND; ++d) P.o[d] = f32x16{};
  P.m = -__builtin_inff();
  P.l = 0.f;
  waitcnt<0, 15>();
  barrier();
  P.template read_k<0>();
  typename PipeT::Sc sa, sb;
  P.qk(sa);
  waitcnt<63, 0>();
  barrier();  // every wave has read K_0: its buffer takes K_2
  if (nte > 2) P.dma_k(2, 0);
  P.dma_v(1, 1);
  if (p.S < PipeT::kBN) P.mask(sa, p.S);  // tile 0 itself ends early
  P.vec0(sa);
  P.vec1(sa);
  P.l *= P.alpha;
  P.template read_k<1>();
  waitcnt<63, 0>();

  const bool lag = wave >= 4;
  stamp(1);
  if (lag) barrier();
  int j = 0;
  for (; j + 2 < nte; j += 2) {
    P.template step<0, true>(j, sa, sb);
    P.template step<1, true>(j + 1, sb, sa);
  }
  P.template step<0, true>(j, sa, sb);
  P.template step<1, false>(j + 1, sb, sa);
  __builtin_amdgcn_s_setprio(0);
  if (!lag) barrier();
  stamp(2);

  const float lt = xhalf(P.l, [](float x, float y) { return x + y; });
  const float inv = 1.f / lt;
  if (qrow < p.S) {
    char* orow = p.o + b * p.o_b + hq * p.o_h + (size_t)qrow * p.ldo;
#pragma unroll
    for (int d = 0; d < PipeT::kND; ++d)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = 32 * d + 8 * r + 4 * h;
        const u32x2 w = {pack2<BF16>(P.o[d][4 * r] * inv, P.o[d][4 * r + 1] * inv),
                         pack2<BF16>(P.o[d][4 * r + 2] * inv, P.o[d][4 * r + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + col * 2) = w;
      }
    if (p.lse && h == 0) p.lse[((size_t)b * p.HQ + hq) * p.S + qrow] = (P.m + __builtin_log2f(lt)) * kLn2;
  }
  stamp(3);
}

}  // namespace fa
}  // namespace g9

using namespace g9;

// Kernels: g9_fmha_fwd_{bf16,f16}_v{3,4}[_d64]; v3 rescales every tile, v4
// lazily; head dim 128, or 64 with the _d64 suffix.
#define G9_FMHA_KERNEL(NAME, BF16, LAZY, HD)                                                              \
  extern "C" __global__ __launch_bounds__(fa::kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void \
  NAME(fa::FaParams p) {                                                                                  \
    __shared__ __attribute__((aligned(1024))) char smem[fa::Pipe<BF16, LAZY, true, HD>::kLdsBytes];        \
    if (p.scale_on_q)                                                                                     \
      fa::fmha_fwd<BF16, LAZY, true, HD>(p, smem);                                                        \
    else                                                                                                  \
      fa::fmha_fwd<BF16, LAZY, false, HD>(p, smem);                                                       \
  }
G9_FMHA_KERNEL(g9_fmha_fwd_bf16_v3, true, false, 128)
G9_FMHA_KERNEL(g9_fmha_fwd_f16_v3, false, false, 128)
G9_FMHA_KERNEL(g9_fmha_fwd_bf16_v4, true, true, 128)
G9_FMHA_KERNEL(g9_fmha_fwd_f16_v4, false, true, 128)
G9_FMHA_KERNEL(g9_fmha_fwd_bf16_v3_d64, true, false, 64)
G9_FMHA_KERNEL(g9_fmha_fwd_f16_v3_d64, false, false, 64)
G9_FMHA_KERNEL(g9_fmha_fwd_bf16_v4_d64, true, true, 64)
G9_FMHA_KERNEL(g9_fmha_fwd_f16_v4_d64, false, true, 64)

extern "C" int g9_fmha_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t HQ,
                           int64_t HK, int64_t S, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                           const int64_t* v_strides, const int64_t* o_strides, float sm_scale, int dtype,
                           int scale_on_q, int variant, void* stream) {
  if (dtype != G9_F16 && dtype != G9_BF16) return G9_ERR_DTYPE;
  if (variant != 3 && variant != 4) return G9_ERR_SCHEDULE;
  if (B <= 0 || HQ <= 0 || HK <= 0 || S <= 0 || HQ % HK != 0) return G9_ERR_SHAPE;
  if ((D != 128 && D != 64) || S % 64 != 0) return G9_ERR_SHAPE;
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return G9_ERR_LAYOUT;
  const int64_t* st[4] = {q_strides, k_strides, v_strides, o_strides};
  const void* ptr[4] = {q, k, v, o};
  for (int i = 0; i < 4; ++i) {
    // (batch, head, seq, dim) strides in elements: unit head-dim stride,
    // 16-byte aligned rows, and every row offset of a (batch, head) slice,
    // including a 256-row tile past the end, inside 31 bits.
    if (st[i][3] != 1 || st[i][2] < D || (st[i][2] * 2) % 16 != 0 || st[i][0] < 0 || st[i][1] < 0) return G9_ERR_LAYOUT;
    if ((uintptr_t)ptr[i] % 16 != 0 || (st[i][0] * 2) % 16 != 0 || (st[i][1] * 2) % 16 != 0) return G9_ERR_LAYOUT;
    if ((S + fa::kBlockM) * st[i][2] * 2 >= (int64_t(1) << 31)) return G9_ERR_SHAPE;
  }
  if (lse && (uintptr_t)lse % 4 != 0) return G9_ERR_LAYOUT;
  const int64_t mblocks = (S + fa::kBlockM - 1) / fa::kBlockM;
  if (B * HQ * mblocks > INT32_MAX) return G9_ERR_SHAPE;
  // This file is compiled without NaN semantics (-fno-honor-nans), under
  // which a float comparison may treat NaN as ordered: the scale's bits are
  // tested instead (a positive, finite, nonzero float).
  const u32 sm_bits = __builtin_bit_cast(u32, sm_scale);
  if ((sm_bits >> 31) != 0 || sm_bits == 0 || ((sm_bits >> 23) & 0xff) == 0xff) return G9_ERR_SHAPE;
  fa::FaParams p{};
  p.q = static_cast<const char*>(q);
  p.k = static_cast<const char*>(k);
  p.v = static_cast<const char*>(v);
  p.o = static_cast<char*>(o);
  p.lse = lse;
  p.q_b = q_strides[0] * 2;
  p.q_h = q_strides[1] * 2;
  p.k_b = k_strides[0] * 2;
  p.k_h = k_strides[1] * 2;
  p.v_b = v_strides[0] * 2;
  p.v_h = v_strides[1] * 2;
  p.o_b = o_strides[0] * 2;
  p.o_h = o_strides[1] * 2;
  p.ldq = (u32)(q_strides[2] * 2);
  p.ldk = (u32)(k_strides[2] * 2);
  p.ldv = (u32)(v_strides[2] * 2);
  p.ldo = (u32)(o_strides[2] * 2);
  p.B = (int)B;
  p.HQ = (int)HQ;
  p.HK = (int)HK;
  p.S = (int)S;
  p.mblocks = (int)mblocks;
  p.num_xcds = 8;
  p.scale_log2 = sm_scale * fa::kLog2e;
  p.scale_on_q = scale_on_q != 0;
  void* args[] = {&p};
  // [head dim 64][lazy][bf16]
  static const void* const kFns[2][2][2] = {
      {{reinterpret_cast<const void*>(g9_fmha_fwd_f16_v3), reinterpret_cast<const void*>(g9_fmha_fwd_bf16_v3)},
       {reinterpret_cast<const void*>(g9_fmha_fwd_f16_v4), reinterpret_cast<const void*>(g9_fmha_fwd_bf16_v4)}},
      {{reinterpret_cast<const void*>(g9_fmha_fwd_f16_v3_d64), reinterpret_cast<const void*>(g9_fmha_fwd_bf16_v3_d64)},
       {reinterpret_cast<const void*>(g9_fmha_fwd_f16_v4_d64), reinterpret_cast<const void*>(g9_fmha_fwd_bf16_v4_d64)}}};
  const void* fn = kFns[D == 64][variant == 4][dtype == G9_BF16];
  return hipLaunchKernel(fn, dim3((unsigned)(B * HQ * mblocks)), dim3(fa::kThreads), args, 0,
                         reinterpret_cast<hipStream_t>(stream)) == hipSuccess
             ? G9_OK
             : G9_ERR_HIP;
}

#ifdef G9_TIMING
#include "../../include/gfx950_gemm_timing.h"
extern "C" int g9_fmha_timing_read(void* host, size_t bytes) {
  if (bytes > sizeof(g9::fa::g9_fmha_timing_buf)) return G9_ERR_SHAPE;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g9::fa::g9_fmha_timing_buf), bytes, 0, hipMemcpyDeviceToHost) ==
                 hipSuccess
             ? G9_OK
             : G9_ERR_HIP;
}
#endif
