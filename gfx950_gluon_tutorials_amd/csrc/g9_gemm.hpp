// NT GEMM kernels for gfx950: C[M,N] = A[M,K] . B[N,K]^T.
//
// One workgroup computes a 256x256 output tile, split into four 128x128
// quadrants.  Two wave geometries share all the code below:
//   * 4-wave (G = Geo4, 1 wave per SIMD): waves 2x2, each owns the 64x64 piece
//     of every quadrant -> 2x2x4x4 MFMA 16x16 fragments x 4 fp32 = 256
//     accumulators per lane (AGPRs).
//   * 8-wave (G = Geo8, 2 waves per SIMD): waves 2x4, each owns a 64x32 piece
//     of every quadrant -> 128 accumulators per lane.  While one wave of a SIMD
//     waits (barrier, counters, DMA issue) the other issues its MFMAs.
//
// K is walked in stages of 128 bytes per operand row: 64 fp16/bf16, 128 bf8 or
// 256 fp4 values.  A stage is split into four LDS sub-buffers of 128 rows x 128
// bytes (A rows 0-127 "A0", A rows 128-255 "A1", B rows 0-127 "B0", B rows
// 128-255 "B1"), each double buffered (two slots), 128 KiB in total.  FP4 adds
// two slots of E8M0 scale chunks (4 stages of every tile row's scales each).
//
// Per stage every wave runs four "quadrant regions" in the order
// Q00 (A0 x B0), Q01 (A0 x B1), Q11 (A1 x B1), Q10 (A1 x B0).  Each region
// issues its MFMAs on operand fragments already in registers, reads the next
// region's operand set from LDS into registers, and refills, by LDS-DMA, a
// sub-buffer every wave has finished reading.  A region starts with
// `s_waitcnt vmcnt(N) lgkmcnt(0)` (N: the DMAs issued since the ones it
// needs), issues its first MFMAs, then `s_barrier`.  With a barrier in every
// region (BF8) a region refills the sub-buffer read in the previous one,
// requested seven regions before it is read again (a DMA latency budget of 1.5
// stages); the other 4-wave kernels pass a barrier in even regions only, and
// refill the sub-buffer read two regions earlier (stage()).  The B operand
// registers alternate roles between even and odd stages, so the loop body
// covers two stages (eight for FP4: two scale chunks).  The 8-wave kernels run
// the same regions in a ping-pong (region_pp).
//
// LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at chunk slot
// c ^ ((r >> 1) & 7).  A ds_read_b128 by 16 consecutive lanes (16 rows, one
// chunk) then touches all 64 banks once.  The LDS-DMA writes each wave's KiB
// contiguously, so the permutation is applied on the global side: lane i
// fetches the chunk that belongs in its slot.
//
// MFMA operands are swapped (the B fragment is the MFMA's A operand), so lane l
// ends with C[m0 + l%16][n0 + 4*(l/16) + 0..3]: four consecutive output
// columns, which the epilogue writes to LDS as one 8-byte store and then streams
// out as coalesced 16-byte row chunks (4-wave: quadrant by quadrant, each
// quadrant's stores beside the next one's conversion).
//
// Three tile schedules drive this pipeline: gemm_dp (one tile per workgroup),
// gemm_sk (persistent workgroups over (tile, stage) ranges with a K-ordered
// fp32 fixup, bit-identical to gemm_dp) and gemm_moe (tiles grouped by
// expert, each expert with its own rows of A and C and its own B).
#pragma once

#include <type_traits>
#include <utility>

#include "g9_common.hpp"

namespace g9 {

// Optional phase stamps (build with -DG9_TIMING; see profiling.py): thread 0
// of each data-parallel workgroup records s_memtime (shader clock) and
// s_memrealtime (100 MHz) at kernel entry, main-loop start, main-loop end and
// kernel end, for the first kTimingTiles workgroups.  Each stamp waits only
// for its own scalar reads, so the pipeline around it is unchanged.  Compiled
// to nothing in the regular build.
#ifdef G9_TIMING
constexpr int kTimingTiles = 16384;
__device__ unsigned long long g9_timing_buf[kTimingTiles * 8];
G9_DEV void timing_stamp(int slot) {
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t = __builtin_amdgcn_s_memtime();
  const unsigned long long r = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_s_waitcnt((63 & 15) | (7 << 4) | (0 << 8) | ((63 >> 4) << 14));  // lgkmcnt(0) only
  if (threadIdx.x == 0 && blockIdx.x < kTimingTiles) {
    g9_timing_buf[blockIdx.x * 8 + slot * 2] = t;
    g9_timing_buf[blockIdx.x * 8 + slot * 2 + 1] = r;
  }
  __builtin_amdgcn_sched_barrier(0);
}
// Stream-K phase accounting (timing build): per persistent workgroup, the
// shader cycles spent waiting for predecessor flags, loading partial tiles
// (until they are in the accumulators) and storing them (until the release
// fence has drained the stores), and how many of each.  Slots: 0/1 clock and
// 100 MHz clock at entry, 2/3 at exit, 4 wait, 5 load, 6 store cycles, 7
// (loads << 32) | stores.
struct SkTimes {
  unsigned long long wait = 0, load = 0, store = 0;
  unsigned nl = 0, ns = 0;
};
G9_DEV unsigned long long clk() {
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t = __builtin_amdgcn_s_memtime();
  __builtin_amdgcn_s_waitcnt((63 & 15) | (7 << 4) | (0 << 8) | ((63 >> 4) << 14));  // lgkmcnt(0) only
  __builtin_amdgcn_sched_barrier(0);
  return t;
}
G9_DEV void sk_stamp(int slot) {
  const unsigned long long t = clk();
  const unsigned long long r = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_s_waitcnt((63 & 15) | (7 << 4) | (0 << 8) | ((63 >> 4) << 14));
  if (threadIdx.x == 0 && blockIdx.x < kTimingTiles) {
    g9_timing_buf[blockIdx.x * 8 + slot] = t;
    g9_timing_buf[blockIdx.x * 8 + slot + 1] = r;
  }
}
G9_DEV void sk_times_store(const SkTimes& t) {
  if (threadIdx.x == 0 && blockIdx.x < kTimingTiles) {
    g9_timing_buf[blockIdx.x * 8 + 4] = t.wait;
    g9_timing_buf[blockIdx.x * 8 + 5] = t.load;
    g9_timing_buf[blockIdx.x * 8 + 6] = t.store;
    g9_timing_buf[blockIdx.x * 8 + 7] = ((unsigned long long)t.nl << 32) | t.ns;
  }
}
#else
G9_DEV void timing_stamp(int) {}
struct SkTimes {};
G9_DEV unsigned long long clk() { return 0; }
G9_DEV void sk_stamp(int) {}
G9_DEV void sk_times_store(const SkTimes&) {}
#endif

// MXFP4 comes with its E8M0 scales in one of three global layouts, all fed
// to the same MFMAs:
//   FP4  row-major (M rows of K/32 bytes): each 4-stage scale chunk lands in
//        LDS as it is in memory and is transposed in place once (see
//        Pipe::xform_read) into the KM layout, 32 rows of all 32 groups per
//        KiB;
//   FP4K K-major (K/32 groups of M bytes, the layout of the reference bench's
//        transposed scale views): the chunk DMA writes the transposed KL
//        layout directly, 8 groups of all 128 rows of a half tile per KiB, so
//        each DMA reads whole 128-byte runs;
//   FP4P preshuffled (quant.preshuffle_e8m0).
// With 16x16 fragments every layout gives a lane all its scale bytes of a
// chunk with one LDS read per fragment (ScRegs) and no byte permute.
enum class Op : int { F16 = 0, BF16 = 1, BF8 = 2, FP4 = 3, FP4P = 4, FP4K = 5 };
enum : int { OUT_F16 = 0, OUT_BF16 = 1 };

struct GemmParams {
  const char* a;              // A: M rows of K-contiguous elements, lda bytes apart
  const char* b;              // B: N rows of K-contiguous elements, ldb bytes apart
  char* c;                    // C: M x N 16-bit values, row stride ldc elements
  const unsigned char* a_sc;  // FP4 only: E8M0 scales, M rows of K/32 bytes, ldsa apart
  const unsigned char* b_sc;  // FP4 only: N rows
  const float* a_scale;       // BF8 only: per-tensor fp32 scales on the device (nullable)
  const float* b_scale;
  int M, N, K;                // K in elements
  u32 lda, ldb;               // operand row strides in bytes
  u32 ldsa, ldsb;             // scale row strides in bytes
  long long ldc;              // C row stride in elements
  int ns;                     // K stages (ceil(K * bits / 1024))
  u32 kshift;                 // K tail: bytes by which stage 0 starts before k = 0 (ns * 128 - K bytes);
                              // the operand resources start that much earlier, stage 0's DMAs zero it
  int tiles_m, tiles_n;
  int num_xcds, group_m;
  // stream-K
  float* ws;                  // fp32 partial tiles (256 KiB per tile)
  u32* flags;                 // one flag per tile: (epoch << 16) | stages done
  u32 epoch;
  int* err;                   // set to 1 when a flag wait times out (workspace header; a host
                              // flag registered at byte 8 of the header is set as well)
  u32 spin_limit;             // polls of a flag wait before it gives up
  int sk_ctas;                // persistent workgroups
  // split-K: K segments per tile (the partials go to ws)
  int split;
  // grouped (MoE) GEMM: expert e owns rows [moe_off[e], moe_off[e+1]) of A
  // and C and its own B (and FP4 B scales) moe_b_stride (moe_bsc_stride)
  // bytes after expert e - 1's
  const int* moe_off;
  int moe_experts;
  long long moe_b_stride, moe_bsc_stride;
};

constexpr int kTile = 256;
constexpr int kRowBytes = 128;              // bytes of one operand row per stage
constexpr int kSubBytes = 128 * kRowBytes;  // one sub-buffer (16 KiB)
constexpr int kStageRow = 528;              // epilogue staging row pitch (bytes; see store_tile)
// FP4 E8M0 scales are staged in chunks of kScChunk stages: one chunk holds
// kScChunk * 8 bytes of each of the tile's 256 A rows and 256 B rows (chunk
// rows 0-255 = A, 256-511 = B), and two chunk slots sit after the operand
// buffers.  A chunk row's 32 bytes are two 16-byte halves (stages 0-1, 2-3);
// rows with bit 3 set store them swapped, so the 16 rows one ds_read_b64
// serves fall on distinct banks.
constexpr int kScaleBase = 131072;
constexpr int kScChunk = 4;
constexpr int kScRowBytes = 8 * kScChunk;
constexpr int kScSlotBytes = 512 * kScRowBytes;  // 16 KiB
// LDS per workgroup: 128 KiB of operand buffers (+ 32 KiB of scale chunks for
// FP4); the epilogue's staging (256 rows x 528 bytes) reuses it.
template <bool SCALED>
constexpr int kLdsBytes = SCALED ? kScaleBase + 2 * kScSlotBytes : kTile * kStageRow;
static_assert(kTile * kStageRow >= kScaleBase && kTile * kStageRow <= kLdsBytes<true>, "staging must fit");

// Wave geometry: NW waves as WM x WN; per quadrant a wave owns FM x FN MFMA
// fragments of MD x MD outputs (FM*MD rows of A, FN*MD rows of B).  A
// fragment's 64 lanes split into NG = 64/MD lane groups: lane l works on row
// l % MD and lane group l / MD, and holds NC = 8/NG of the eight 16-byte chunks
// of that row in a stage.
template <int NW_, int WM_, int WN_, int MD_>
struct Geo {
  static constexpr int NW = NW_, WM = WM_, WN = WN_, MD = MD_;
  static_assert(MD == 16 || MD == 32, "MFMA fragments are 16x16 or 32x32");
  static constexpr int kThreads = 64 * NW;
  static constexpr int FM = 128 / WM / MD, FN = 128 / WN / MD;
  static constexpr int FMAX = FM > FN ? FM : FN;
  static constexpr int NG = 64 / MD;        // lane groups per fragment
  static constexpr int NC = 8 / NG;         // 16-byte chunks per lane per fragment per stage
  static constexpr int NB = MD * MD / 256;  // 4-float accumulator quads per fragment
  static constexpr int kDmaRows = 128 / NW;        // rows of each sub-buffer one wave loads
  static constexpr int kDmaPerSub = kDmaRows / 8;  // 16-byte DMAs per wave per sub-buffer
  // FP4 scale chunks: each wave loads 512 / NW chunk rows as kScParts
  // 16-byte DMAs of 32 rows x 32 bytes.
  static constexpr int kScRows = 512 / NW;
  static constexpr int kScParts = kScRows / 32;
  static constexpr int kWavesPerSimd = NW / 4;
  // Row chunk held as the lane's chunk r by lane group gi.  The same map is
  // used for A and B, so it only permutes K inside a stage.
  //   MD 16: chunk 4r + gi.  16x16 MFMA step r takes K chunk 4r..4r+3 from
  //          lane groups 0..3, which is the natural K order for FP16/BF16/FP4;
  //          BF8 feeds chunks r = 0, 1 to one MFMA (a K permutation), which
  //          keeps the read pattern of the 16-bit types, free of bank
  //          conflicts (the contiguous chunks 2gi, 2gi + 1 measured 2-way
  //          conflicts).
  //   MD 32: chunk 4gi + r.  Lane group gi holds K chunks 4gi..4gi+3, so an
  //          FP4 lane's four E8M0 scales (groups 4gi..4gi+3) are one aligned
  //          dword of its row's eight scale bytes, read without a byte
  //          shuffle.
  static constexpr int chunk(int r, int gi) { return MD == 16 ? 4 * r + gi : 4 * gi + r; }
};
template <int MD>
using Geo4 = Geo<4, 2, 2, MD>;
template <int MD>
using Geo8 = Geo<8, 2, 4, MD>;

// MFMA fragment size per operand type (build-time choice, 16 or 32).  32x32
// MFMAs are twice as long as the 16x16 ones, which leaves more issue slots per
// MFMA for the LDS reads, DMAs and barrier (a block-scaled 16x16x128 MFMA
// leaves only one) and halves the number of block-scale loads: the loop runs
// at 97-98% MFMA occupancy for FP16/BF8 and 87% for MXFP4, against 90%, 96%
// and 73% with 16x16.  But the chip is power-limited in this kernel, the
// 32x32 MFMAs draw more energy per FLOP, and the sustained clock drops by more
// than the occupancy gains: measured back to back on the same MI355X at
// 4096x4096x8192, 16x16 is 6% faster for FP16, 5% for BF8 and 1.5% for MXFP4.
#ifndef G9_MD_F16
#define G9_MD_F16 16
#endif
#ifndef G9_MD_BF8
#define G9_MD_BF8 16
#endif
#ifndef G9_MD_FP4
#define G9_MD_FP4 16
#endif

// Operand fragment of one MD-row slice for one stage: NC chunks of 16 bytes
// per lane, plus (FP4) the lane's E8M0 scales.
template <int NC>
struct Frag {
  u32x4 c[NC];
  u32x2 sc;  // FP4, MD 16: the lane's 8 raw E8M0 bytes of the stage (groups 0..7)
  u32 sp;    // FP4: byte e = scale of the lane's data in MFMA step e
};

template <Op OP>
struct OpInfo {
  static constexpr bool kScaled = OP == Op::FP4 || OP == Op::FP4P || OP == Op::FP4K;
  static constexpr bool kPreshuffled = OP == Op::FP4P;
  static constexpr bool kKMajor = OP == Op::FP4K;
  static constexpr int kChunksPerMfma = OP == Op::BF8 ? 2 : 1;  // 16-byte chunks per lane per MFMA
};
template <Op OP>
constexpr int kMfmaDim = OP == Op::BF8 ? G9_MD_BF8 : OP == Op::FP4 ? G9_MD_FP4 : OP == Op::FP4P || OP == Op::FP4K ? 16 : G9_MD_F16;
// The 8-wave MXFP4 kernel uses 32x32x64 fragments: with 16x16 ones its
// operand sets, scale bytes and DMA offsets exceed the 128 VGPRs a wave has
// beside its accumulators at 2 waves per SIMD, and the spill reloads inside
// the loop (VMEM loads, retired in order behind the DMAs) drain the pipeline.
#ifndef G9_MD_FP4_8W
#define G9_MD_FP4_8W 32
#endif
template <Op OP>
constexpr int kMfmaDim8 = OP == Op::FP4 || OP == Op::FP4P ? G9_MD_FP4_8W : kMfmaDim<OP>;

// Scale paths of the scaled kernels:
//  * kTrScales: chunks in LDS in a transposed layout (KM for FP4, KL for
//    FP4K), read with ds_read_b64_tr_b8 -- FP4 and FP4K with 16x16
//    fragments and 4 waves;
//  * kXform: FP4 of those, whose row-major chunks are transposed in place;
//  * kChunkScales: a lane reads all its scale bytes of a chunk at once into
//    ScRegs (kTrScales and FP4P).  The other FP4 kernels (8 waves with 32x32
//    fragments) read one scale word per fragment and stage from row-major
//    chunks.
template <Op OP, class G>
constexpr bool kTrScales = (OP == Op::FP4 || OP == Op::FP4K) && G::MD == 16 && G::NW == 4;
template <Op OP, class G>
constexpr bool kXform = OP == Op::FP4 && kTrScales<OP, G>;
template <Op OP, class G>
constexpr bool kChunkScales = OP == Op::FP4P || kTrScales<OP, G>;

// Per-region work and the DMA pattern of the main loop.  The loop body covers
// kBody stages = 4 * kBody regions, numbered by their body position.  Every
// region issues kDmaPerSub operand DMAs per wave.  FP4 adds the scale-chunk
// DMAs: with a body of two chunks (8 stages), a chunk's kScParts parts are
// issued at positions 16h + 14 (part 0 of the chunk two ahead of chunk h) and
// 16h + 0, 2, 4 (the remaining parts of the chunk one ahead), each at least
// 10 regions before the chunk is first read (position 16h + 14 reads the next
// chunk's first stage) and after the slot's previous chunk was last read
// (position 16h + 13); all of these positions are even, so each has a
// barrier under either barrier pattern.  With a barrier per region, a region
// waits for the DMAs issued 7 regions earlier: vmcnt(number of DMAs issued in
// the 6 regions between), a constant per body position because the pattern
// repeats every 16 regions (vm_wait_hb: the half-barrier pattern).
template <Op OP, class G>
struct Shape {
  static constexpr int KS = G::NC / OpInfo<OP>::kChunksPerMfma;  // MFMA steps per stage
  static constexpr int NM = G::FM * G::FN * KS;                  // MFMAs per wave per region
  static constexpr bool kScaled = OpInfo<OP>::kScaled;
  static constexpr int kBody = kScaled ? 2 * kScChunk : 2;       // stages per loop iteration
  static constexpr int kRegions = 4 * kBody;
  static constexpr int D = G::kDmaPerSub;
  // Scale-chunk part issued at body position `pos`, or -1.
  static constexpr int sc_part(int pos) {
    if (!kScaled) return -1;
    const int q = pos % 16;
    if (q == 14) return 0;
    if (q % 2 == 0 && q / 2 + 1 < G::kScParts) return q / 2 + 1;
    return -1;
  }
  static constexpr int dmas(int pos) { return D + (sc_part(pos) >= 0 ? 1 : 0); }
  static constexpr int vm_wait(int pos) {
    int n = 0;
    for (int q = 1; q <= 6; ++q) n += dmas(((pos - q) % kRegions + kRegions) % kRegions);
    return n;
  }
  // Ping-pong (8-wave): at the end of region pos's memory cluster, the DMAs
  // issued 6 regions earlier must have landed (the next memory cluster reads
  // them, and the other wave group reads them one cluster later still):
  // vmcnt(DMAs of region pos and the 5 before it).
  static constexpr int vm_wait_pp(int pos) {
    int n = 0;
    for (int q = 0; q <= 5; ++q) n += dmas(((pos - q) % kRegions + kRegions) % kRegions);
    return n;
  }
  // Barriers at even positions only (kHalfBarrier): an even region's barrier
  // also publishes the data the next (odd) region reads, so it waits for the
  // DMAs issued 5 regions earlier: vmcnt(DMAs of the 4 regions between).
  static constexpr int vm_wait_hb(int pos) {
    int n = 0;
    for (int q = 1; q <= 4; ++q) n += dmas(((pos - q) % kRegions + kRegions) % kRegions);
    return n;
  }
  static_assert(vm_wait(0) < 64 && vm_wait_pp(0) < 64, "vmcnt is 6 bits");
};

template <class G>
using accv = std::conditional_t<G::MD == 16, f32x4, f32x16>;
template <class G>
using FragSet = Frag<G::NC>[G::FMAX];

// Four consecutive accumulator registers 4B..4B+3 of a fragment.
template <int B, class V>
G9_DEV f32x4 get_quad(const V& v) {
  if constexpr (sizeof(V) == sizeof(f32x4))
    return v;
  else
    return __builtin_shufflevector(v, v, 4 * B, 4 * B + 1, 4 * B + 2, 4 * B + 3);
}
// A fragment's accumulators from NB quads (p[0], p[64], ... : one quad per
// 64-lane row of a partial tile).
template <class V>
G9_DEV V load_quads(const f32x4* p) {
  if constexpr (sizeof(V) == sizeof(f32x4)) {
    return p[0];
  } else {
    const f32x4 a = p[0], b = p[64], c = p[128], d = p[192];
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7),
                                   __builtin_shufflevector(c, d, 0, 1, 2, 3, 4, 5, 6, 7), 0, 1, 2, 3, 4, 5, 6, 7, 8,
                                   9, 10, 11, 12, 13, 14, 15);
  }
}

// LDS byte offset of operand sub-buffer X (0:A0 1:A1 2:B0 3:B1) in slot s.
constexpr int sub_off(int X, int s) { return (X >> 1) * 65536 + ((X & 1) * 2 + s) * kSubBytes; }

// Block-scaled e2m1 x e2m1 MFMA (format code 4) whose scales are byte BYTE of
// sx (for x, the MFMA's first operand) and of sy: op_sel and op_sel_hi bit 0
// of the scale operands select the byte.
#define G9_MFMA_SCALED_ASM(SHAPE, SEL)                                                               \
  asm("v_mfma_scale_f32_" SHAPE "_f8f6f4 %0, %1, %2, %0, %3, %4 " SEL " cbsz:4 blgp:4"              \
      : "+a"(acc)                                                                                 \
      : "v"(x), "v"(y), "v"(sx), "v"(sy))
template <int BYTE, class ACC>
G9_DEV void mfma_scaled(ACC& acc, const u32x4& x, const u32x4& y, u32 sx, u32 sy) {
  static_assert(BYTE >= 0 && BYTE < 4, "a scale VGPR holds four bytes");
  if constexpr (sizeof(ACC) == sizeof(f32x4)) {
    if constexpr (BYTE == 0)
      G9_MFMA_SCALED_ASM("16x16x128", "op_sel_hi:[0,0,0]");
    else if constexpr (BYTE == 1)
      G9_MFMA_SCALED_ASM("16x16x128", "op_sel:[1,1,0] op_sel_hi:[0,0,0]");
    else if constexpr (BYTE == 2)
      G9_MFMA_SCALED_ASM("16x16x128", "op_sel_hi:[1,1,0]");
    else
      G9_MFMA_SCALED_ASM("16x16x128", "op_sel:[1,1,0] op_sel_hi:[1,1,0]");
  } else {
    if constexpr (BYTE == 0)
      G9_MFMA_SCALED_ASM("32x32x64", "op_sel_hi:[0,0,0]");
    else if constexpr (BYTE == 1)
      G9_MFMA_SCALED_ASM("32x32x64", "op_sel:[1,1,0] op_sel_hi:[0,0,0]");
    else if constexpr (BYTE == 2)
      G9_MFMA_SCALED_ASM("32x32x64", "op_sel_hi:[1,1,0]");
    else
      G9_MFMA_SCALED_ASM("32x32x64", "op_sel:[1,1,0] op_sel_hi:[1,1,0]");
  }
}
#undef G9_MFMA_SCALED_ASM

// MFMA step E of the stage on a (B fragment, A fragment) pair, written as
// inline assembly with the accumulator tied in place ("+a").  The compiler
// selects an untied MFMA form for the builtins and then renames every
// accumulator chain across the AGPRs, which costs hundreds of AGPR copies per
// loop iteration; the tied form keeps each chain in its registers.  The
// hazard recognizer does not see through inline assembly, so the callers
// insert the MFMA-to-VALU wait states themselves (see mfma_drain) and never
// feed an MFMA from a VALU result written within a few cycles.  (Back-to-back
// MFMAs accumulating into the same registers need no wait states.)
template <Op OP, class G, int E>
G9_DEV void mma(accv<G>& acc, const Frag<G::NC>& bx, const Frag<G::NC>& ay) {
  static_assert(OP != Op::FP4P, "preshuffled-scale MFMAs take their scales from ScRegs");
  if constexpr (G::MD == 16) {
    if constexpr (OP == Op::F16) {
      asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(bx.c[E]), "v"(ay.c[E]));
    } else if constexpr (OP == Op::BF16) {
      asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(bx.c[E]), "v"(ay.c[E]));
    } else if constexpr (OP == Op::BF8) {
      // e5m2 x e5m2 (format code 1), 32 bytes per lane; no block scales (the
      // per-tensor scales are applied in the epilogue).
      const i32x8 x = __builtin_bit_cast(i32x8, __builtin_shufflevector(bx.c[0], bx.c[1], 0, 1, 2, 3, 4, 5, 6, 7));
      const i32x8 y = __builtin_bit_cast(i32x8, __builtin_shufflevector(ay.c[0], ay.c[1], 0, 1, 2, 3, 4, 5, 6, 7));
      asm("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0 cbsz:1 blgp:1" : "+a"(acc) : "v"(x), "v"(y));
    } else {
      // e2m1 x e2m1, 16 bytes per lane; step E's scales are byte E of sp.
      mfma_scaled<E>(acc, bx.c[E], ay.c[E], bx.sp, ay.sp);
    }
  } else {
    if constexpr (OP == Op::F16) {
      asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(bx.c[E]), "v"(ay.c[E]));
    } else if constexpr (OP == Op::BF16) {
      asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(bx.c[E]), "v"(ay.c[E]));
    } else if constexpr (OP == Op::BF8) {
      const i32x8 x =
          __builtin_bit_cast(i32x8, __builtin_shufflevector(bx.c[2 * E], bx.c[2 * E + 1], 0, 1, 2, 3, 4, 5, 6, 7));
      const i32x8 y =
          __builtin_bit_cast(i32x8, __builtin_shufflevector(ay.c[2 * E], ay.c[2 * E + 1], 0, 1, 2, 3, 4, 5, 6, 7));
      asm("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0 cbsz:1 blgp:1" : "+a"(acc) : "v"(x), "v"(y));
    } else {
      mfma_scaled<E>(acc, bx.c[E], ay.c[E], bx.sp, ay.sp);
    }
  }
}

// Wait states between the last inline-assembly MFMA writing an accumulator and
// the first VALU/memory access to it (the longest gfx950 MFMA here, the 32x32
// BF8 one, needs 20).
G9_DEV void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <int N, class F>
G9_DEV void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) { (f(std::integral_constant<int, I>{}), ...); }(
      std::make_integer_sequence<int, N>{});
}

// Where, inside a region of NM MFMAs, the other instructions are issued.  The
// first kPre MFMAs are issued before the region's s_barrier (their operands
// are already in registers), so the MFMA pipe stays busy while the barrier
// resolves; everything else follows the barrier, placed after MFMA kPre + q
// for q in [0, NQ).  The region's NR 16-byte LDS reads come first, spread over
// a window of W slots, so the region-closing lgkmcnt(0) finds them complete;
// the DMAs are spread over the whole region.  FP4 reads one scale word per
// fragment after the first reads; with 16x16 fragments it then gathers the
// bytes each MFMA step needs, one fragment per slot in the slots perm_q(F)
// just before the region's last (a block-scaled MFMA leaves one issue slot
// beside it, so four permutes in one slot held up the MFMA stream: spreading
// them measured ~1% faster), after the reads and before the next region's
// MFMAs read the results.
template <Op OP, class G, int NF>
struct Slots {
  static constexpr int NM = Shape<OP, G>::NM;
  static constexpr int kPre = (G::MD == 32 || OP == Op::BF8 || G::NW == 8) ? 1 : 2;
  static constexpr int NQ = NM - kPre;
  static constexpr int NR = G::NC * NF;
  static constexpr int W = NQ < (NR > NQ / 2 ? NR : NQ / 2) ? NQ : (NR > NQ / 2 ? NR : NQ / 2);
  static constexpr int read_q(int R) { return R * W / NR; }
  static constexpr int kScaleStep = (W + NF - 1) / NF;
  static constexpr int scale_q(int F) { return 1 + F * kScaleStep; }
  static constexpr int D = G::kDmaPerSub;
  static constexpr int dma_q(int J) { return NQ == 1 ? 0 : 1 + J * (NQ - 1) / D; }
  static constexpr int kScaleDmaQ = dma_q(D - 1) + 2 < NQ ? dma_q(D - 1) + 2 : NQ - 1;
  static constexpr int kLastQ = (read_q(NR - 1) > scale_q(NF - 1) ? read_q(NR - 1) : scale_q(NF - 1)) + 3;
  static constexpr int perm_q(int F) { return NQ - NF - 1 + F; }
  // kXform: slot of a region's transpose reads or writes (after the
  // operand reads, between the operand DMAs).
#ifndef G9_XFORM_Q
#define G9_XFORM_Q 17
#endif
  static constexpr int kXformQ = G9_XFORM_Q < NQ ? G9_XFORM_Q : NQ - 1;
  static_assert(NQ >= 1, "a region needs an MFMA after its barrier");
  static_assert(!OpInfo<OP>::kScaled || scale_q(NF - 1) < NQ, "scale reads must fit the region");
  static_assert(!OpInfo<OP>::kScaled || kChunkScales<OP, G> || G::MD != 16 || perm_q(0) >= kLastQ,
                "permutes must follow the scale reads");
};

// Keeps a value in a register the compiler cannot see through, so constant
// parts of LDS addresses stay in the instruction's offset field.
G9_DEV u32 opaque(u32 x) {
  asm volatile("" : "+v"(x));
  return x;
}
// Same for a wave-uniform value, which also keeps the compiler from hoisting
// everything derived from it out of the loop.
G9_DEV u32 opaque_s(u32 x) {
  asm volatile("" : "+s"(x));
  return x;
}
// The thread's index, formed afresh where a tile's set-up starts: the wave's
// base index is an SGPR (lane 0's threadIdx.x, read once) and the lane comes
// from mbcnt, so no VGPR holds threadIdx.x for the whole kernel, and the
// per-lane addresses derived from it are recomputed for every stream-K
// segment instead of being hoisted out of the persistent loop, where the
// dozens of them outlived the registers and were spilled.
// A persistent kernel reads the wave's base once, before its loop, and
// passes it in as `wb` (threadIdx.x read inside the loop would keep the raw
// index register alive through it).
G9_DEV int fresh_tid_at(int base) {
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  return base + lane;
}
G9_DEV int fresh_tid(int wb = -1) {
  return fresh_tid_at(wb >= 0 ? wb : __builtin_amdgcn_readfirstlane(threadIdx.x));
}

// SGPR offset of a DMA for a stage past the end of K: the buffer range check
// covers voffset + soffset + imm, every resource holds at most 2^31 bytes
// (128 rows x a row stride of at most 2^24) and voffset + imm stays below
// 2^31, so the access is out of range (it reads zeros, without memory
// traffic) and the sum does not wrap.
constexpr u32 kDeadOff = 0x80000000u;

// ds_read_b64_tr_b8 at LDS address addr + IMM (see Pipe::init for its lane
// map), and a 16-byte LDS store.  Both are inline assembly: the compiler
// cannot tell a transpose read of the scale chunks from the LDS-DMA writes
// in flight and would put a vmcnt(0) wait before each one (measured in the
// built code), and the stores that complete a transpose must stay ordered
// with those reads.  The compiler does not wait for the read's result
// either: every use comes after a region-start lgkmcnt(0), and isa_check.py
// proves on the built code that nothing touches the destination earlier.
template <int IMM>
G9_DEV u32x2 tr_read(u32 addr) {
  static_assert(IMM >= 0 && IMM < 65536, "DS offsets are 16 bits");
  u32x2 v;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(IMM) : "memory");
  return v;
}
template <int IMM>
G9_DEV void lds_store16(u32 addr, u32x2 lo, u32x2 hi) {
  static_assert(IMM >= 0 && IMM < 65536, "DS offsets are 16 bits");
  const u32x4 v = {lo.x, lo.y, hi.x, hi.y};
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(IMM) : "memory");
}

// kChunkScales: a wave's E8M0 scales of one chunk (four stages), one u32x2
// per fragment: .x holds stages 0-1 and .y stages 2-3, byte 2 * (stage & 1) +
// step of each.  A fragment set's scales are read when the region that reads
// its operands reaches the chunk's first stage.  B0 is used in a stage's
// first and last regions, so its last use in one chunk and its first in the
// next are adjacent regions; its registers alternate by chunk parity.  The
// other sets have two regions between those uses and are overwritten in
// place.  kXform adds the two transposed units of the part being transposed,
// held from the region that reads them to the region that writes them back.
template <Op OP, class G, bool = kChunkScales<OP, G>>
struct ScRegs {};
template <Op OP, class G>
struct ScRegs<OP, G, true> {
  static_assert(G::MD == 16, "chunk scales are read for 16x16 fragments");
  u32x2 a[2][G::FM];   // A0, A1
  u32x2 b1[G::FN];
  u32x2 b0[2][G::FN];  // B0, by chunk parity
  u32x2 t[2];          // kXform
};

// Per-workgroup pipeline state: buffer resources, per-lane DMA offsets and LDS
// read bases.  One instance per output tile (rebuilt per stream-K segment).
template <Op OP, class G>
struct Pipe {
  using I = OpInfo<OP>;
  static_assert(!I::kKMajor || kTrScales<OP, G>, "K-major scales are read by the 4-wave 16x16 kernels");
  static constexpr int D = G::kDmaPerSub;
  static constexpr int SP = I::kScaled ? G::kScParts : 1;
  rsrc_t rA[2], rB[2];      // operand half-tiles
  rsrc_t rS;                // FP4: the scale rows this wave loads into the chunks
  u32 vA[D], vB[D];         // DMA offsets of the wave's 1-KiB runs
  u32 vS[SP];               // FP4: chunk DMA offsets (32 rows x 32 bytes each)
  u32 bA[G::NC], bB[G::NC];  // LDS read bases of the lane's chunks (A at 0, B at 64 KiB)
  u32 bS[2][2];             // FP4: LDS read bases [A/B][stages 0-1 / 2-3 of a chunk] (kTrScales:
                            // [A/B][fragment parity])
  u32 tb[2], tw;            // kXform: LDS bases of the transpose's reads and writes
  u32 sel;                  // FP4, MD 16: scale byte selector
  u32 cstride;              // FP4P: bytes between consecutive scale chunks of this wave's operand;
                            // FP4K: bytes between consecutive scale groups
  u32 lds0;                 // LDS address of the shared buffer
  u32 mrow;                 // LDS address of the wave's rows in sub-buffer A0, slot 0
  u32 msc;                  // FP4: LDS address of the wave's chunk rows in chunk slot 0
  int wave;
  int s0;                   // first stage of the range (chunks are counted from here)
  int s_end;                // first stage not to load
  u32 kshift;               // GemmParams::kshift

  G9_DEV void init(const GemmParams& p, char* smem, int tm, int tn, int first, int end, int wb = -1) {
    // Tile coordinates are wave-uniform; saying so keeps the buffer resources
    // in SGPRs (a resource the compiler thinks divergent is issued through a
    // per-lane "waterfall" loop around every DMA).
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    s0 = __builtin_amdgcn_readfirstlane(first);
    s_end = __builtin_amdgcn_readfirstlane(end);
    kshift = p.kshift;
    lds0 = (u32)(uintptr_t)to_lds(smem);
    const int tid = fresh_tid(wb);
    const int lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    mrow = lds0 + (u32)wave * (G::kDmaRows * kRowBytes);
    const int wm = wave / G::WN, wn = wave % G::WN;
    const int gi = lane / G::MD, rr = lane % G::MD;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ra = tm * kTile + h * 128, rb = tn * kTile + h * 128;
      // Valid rows (the clamp is a VALU med3): stated uniform, so the
      // resources stay in SGPRs.
      const int va = __builtin_amdgcn_readfirstlane(min(max(p.M - ra, 0), 128));
      const int vb = __builtin_amdgcn_readfirstlane(min(max(p.N - rb, 0), 128));
      // A K tail shifts every stage by kshift bytes: stage s covers row bytes
      // [128 s - kshift, 128 (s + 1) - kshift), so the base moves back by
      // kshift (and the valid range grows by it) while the DMA offsets stay
      // 128 s + chunk; stage 0's chunks before k = 0 are zeroed (issue()).
      rA[h] = make_rsrc(p.a + (size_t)ra * p.lda - p.kshift, (u32)va * p.lda + p.kshift);
      rB[h] = make_rsrc(p.b + (size_t)rb * p.ldb - p.kshift, (u32)vb * p.ldb + p.kshift);
    }
    // DMA j of a sub-buffer covers rows 8j..8j+7 of the wave's share and is
    // issued with immediate offset 1024j, which advances the LDS destination
    // by 1024j as well, so the four DMAs of a region share one M0.  The global
    // offset gives the 1024j back (row >= 8j and lda >= 128, so it stays
    // non-negative); the buffer range check sees voffset + soffset + imm, i.e.
    // the row's true offset, so rows past the valid count still read zero.
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int row = G::kDmaRows * wave + 8 * j + (lane >> 3);
      const int ch = (lane & 7) ^ ((row >> 1) & 7);
      vA[j] = (u32)row * p.lda + ch * 16 - 1024u * j;
      vB[j] = (u32)row * p.ldb + ch * 16 - 1024u * j;
    }
    // Fragment row bases are multiples of 16, so the swizzle of the lane's
    // row depends on rr only.
    const int sw = (rr >> 1) & 7;
#pragma unroll
    for (int c = 0; c < G::NC; ++c) {
      const int slot = G::chunk(c, gi) ^ sw;
      bA[c] = opaque(lds0 + (u32)(wm * G::FM * G::MD + rr) * kRowBytes + slot * 16);
      bB[c] = opaque(lds0 + 65536u + (u32)(wn * G::FN * G::MD + rr) * kRowBytes + slot * 16);
    }
    if constexpr (I::kPreshuffled) {
      // Preshuffled scales (quant.preshuffle_e8m0): chunk c (stages 4c..4c+3)
      // of row r is 32 bytes at c * cstride + r * 32, byte 8j + 2st + h being
      // the scale of group 8st + 4h + g (lane group g = j ^ ((r >> 2) & 3),
      // stage st of the chunk, MFMA step h).  A chunk part of 32 rows is one contiguous KiB, so every
      // part DMA shares one offset and moves by 1024 bytes through its
      // immediate, in global memory and LDS alike.  The resource covers the
      // operand's whole scale array; rows past the end in the last chunk read
      // zero, rows past the end in earlier chunks read the next chunk's rows
      // (they only meet A or B rows that read zero and outputs that are not
      // stored).  The LDS chunk slot holds the tile's 512 rows of 32 bytes in
      // the same order, and lane (row, g) reads its 8 bytes at row * 32 +
      // 8 * (g ^ ((row >> 2) & 3)): the XOR puts the 16 rows of a read pass
      // on distinct bank pairs (without it rows r and r + 4 share one: 2-way
      // conflicts, measured).  Fragment rows start at multiples of 16, so the
      // XOR depends on the lane's row rr only.
      const int xw = wave / (G::NW / 4);
      const int r0 = (wave % (G::NW / 4)) * G::kScRows;
      const bool sa = xw < 2;
      cstride = __builtin_amdgcn_readfirstlane(sa ? p.ldsa : p.ldsb);
      const int rows = sa ? p.M : p.N;
      const u32 nchunks = (u32)(p.ns + kScChunk - 1) / kScChunk;
      rS = make_rsrc(sa ? p.a_sc : p.b_sc, (nchunks - 1) * cstride + (u32)rows * kScRowBytes);
      const int hrow = (sa ? tm : tn) * kTile + (xw & 1) * 128;
      vS[0] = (u32)(hrow + r0) * kScRowBytes + 16u * lane;
      msc = lds0 + kScaleBase + (u32)(xw * 128 + r0) * kScRowBytes;
      const u32 unit = 8u * (u32)(gi ^ ((rr >> 2) & 3));
      bS[0][0] = opaque(lds0 + kScaleBase + (u32)(wm * G::FM * G::MD + rr) * kScRowBytes + unit);
      bS[1][0] = opaque(lds0 + kScaleBase + (u32)(256 + wn * G::FN * G::MD + rr) * kScRowBytes + unit);
      sel = 0;
    } else if constexpr (I::kScaled) {
      // The wave loads chunk rows [xw * 128 + r0, + kScRows) of the 512: half
      // tile xw (0: A0, 1: A1, 2: B0, 3: B1), rows r0.. of it, as kScParts
      // 1-KiB parts of 32 rows.
      // The resource is built from wave-uniform scalars (a select between
      // prebuilt resources is lowered through VGPRs, which turns every DMA
      // into a per-lane loop).
      const int xw = wave / (G::NW / 4);
      const int r0 = (wave % (G::NW / 4)) * G::kScRows;
      const bool sa = xw < 2;
      const u32 lds = sa ? p.ldsa : p.ldsb;
      const int hrow = (sa ? tm : tn) * kTile + (xw & 1) * 128;
      const int hvalid = __builtin_amdgcn_readfirstlane(min(max((sa ? p.M : p.N) - hrow, 0), 128));
      msc = lds0 + kScaleBase + (u32)(xw * 128 + r0) * kScRowBytes;
      if constexpr (I::kKMajor) {
        // K-major scales: group q of the operand at q * lds, rows contiguous.
        // The chunk's KL layout (below) is written directly: lane l of part j
        // fills unit position l & 7 of group row G = 8 j + l / 8, i.e. the 16
        // rows 16 u .. of u = (l & 7) ^ (G >> 2), so the eight lanes of a
        // group row fetch its 128 contiguous bytes and a part reads eight
        // whole 128-byte runs.  Rows past the operand's end read the next
        // group's first rows (scales of A or B rows that read zero, whose
        // outputs are not stored) or, in the last group, zero.
        cstride = __builtin_amdgcn_readfirstlane(lds);
        const u32 groups = (u32)p.K / 32;
        rS = make_rsrc((sa ? p.a_sc : p.b_sc) + hrow, (groups - 1) * lds + (u32)hvalid);
#pragma unroll
        for (int j = 0; j < SP; ++j) {
          const int grp = 8 * j + (lane >> 3);
          vS[j] = (u32)grp * lds + 16u * (u32)((lane & 7) ^ (grp >> 2));
        }
      } else {
        // Row-major scales: lane l of part j fetches the 16-byte half of row
        // 32 j + l / 2 that belongs in its LDS half under the bit-3 row swap.
        const unsigned char* hbase = (sa ? p.a_sc : p.b_sc) + (size_t)hrow * lds;
        rS = make_rsrc(hbase, (u32)hvalid * lds);
#pragma unroll
        for (int j = 0; j < SP; ++j) {
          const int row = r0 + 32 * j + (lane >> 1);
          const int half = (lane & 1) ^ ((row >> 3) & 1);
          vS[j] = (u32)row * lds + half * 16;
        }
      }
      if constexpr (I::kKMajor) {
        // KL layout of a chunk slot (K-major scales): half tile X at X *
        // 4096, group G (0..31) at + 128 G, the 16-byte unit of its rows
        // 16 u .. 16 u + 15 at + 16 (u ^ (G >> 2)).  ds_read_b64_tr_b8
        // gives lane 8a + b of each 16-lane group byte b of the 8-byte units
        // addressed by lanes a, a + 2, ..., a + 14 of the group (measured on
        // gfx950).  For fragment F (rows 16 u .. of u = 4 wm + F) lane 16g +
        // 2k + a addresses the half a of unit (group 4k + g, u), so lane (g,
        // row rr) receives the scales of its row for groups g, 4 + g, ...,
        // 28 + g: byte 2 st + h is stage st, MFMA step h, as the MFMAs take
        // them.  The address of fragment F is fragment 0's with bits 4-5
        // XORed with F (the unit index is u ^ k and F < 4 only touches its
        // low bits).  Per 32 lanes (two lane groups: group rows of both
        // parities, eight unit positions, two halves) the 32 units sit on 64
        // distinct banks.
        const int g = lane >> 4, k = (lane >> 1) & 7, a = lane & 1;
        const u32 off = 128u * (u32)(4 * k + g) + 8u * (u32)a;
        bS[0][0] = opaque(lds0 + kScaleBase + off + 16u * (u32)((4 * wm) ^ k));
        bS[1][0] = opaque(lds0 + kScaleBase + 8192u + off + 16u * (u32)((4 * wn) ^ k));
        sel = 0;
      } else if constexpr (kTrScales<OP, G>) {
        // KM layout of a chunk slot: half tile X at X * 4096, its part jj
        // (rows 32 jj .. 32 jj + 31) at + jj * 1024; in a part, group G
        // (0..31) is a 32-byte row at position p(G) = ((G >> 2) ^ (G & 2)) +
        // 8 (G & 3), holding the part's four 8-row octets, octet o at
        // 8 (o ^ 2 (G & 1)): the scales of rows 8o .. 8o + 7, in row order.
        // ds_read_b64_tr_b8 gives lane 8a + b of each 16-lane group byte b of
        // the 8-byte units addressed by lanes a, a + 2, ..., a + 14 of the
        // group (measured on gfx950).  Lane 16g + 2k + a addresses the unit
        // of group 4k + g and octet a of the fragment's two, so lane (g, row
        // rr) receives the scales of its row for groups g, 4 + g, ..., 28 + g:
        // byte 2 st + h is stage st, MFMA step h, as the MFMAs take them.
        // Per 32 lanes (two lane groups, one value of g & 2) the 16 units sit
        // on 64 distinct banks.  The XOR of G & 2 in p(G) is for the
        // transpose's writes below: without it the two lanes of a write pass
        // whose groups differ only in bit 1 hit the same banks (measured,
        // 1152 conflict cycles per workgroup).
        const int g = lane >> 4, k = (lane >> 1) & 7, a = lane & 1;
#pragma unroll
        for (int f2 = 0; f2 < 2; ++f2) {
          const u32 off = 32u * (u32)((k ^ (g & 2)) + 8 * g) + 8u * (u32)((2 * f2 + a) ^ (2 * (g & 1)));
          bS[0][f2] = opaque(lds0 + kScaleBase + (u32)wm * 2048u + off);
          bS[1][f2] = opaque(lds0 + kScaleBase + 8192u + (u32)wn * 2048u + off);
        }
        if constexpr (kXform<OP, G>) {
          // In-place transpose of a row-major part (32 rows x 32 bytes, the
          // halves of rows with bit 3 set swapped).  In read i (0, 1), lane
          // 16g + 2k + a addresses row 8 (2a + i) + k, groups 8u .. 8u + 7 of
          // u = g ^ 2a, so lane 16g + 8a + b receives the KM unit of group
          // 8 (g ^ 2a) + b, octet 2a + i.  Its two units are adjacent in the
          // KM layout and go back with one 16-byte write once both reads of
          // the part have landed.  The reads put 32 lanes on 64 distinct
          // banks (rows 8 apart differ in the half swap, u >> 1 follows a).
#pragma unroll
          for (int i = 0; i < 2; ++i)
            tb[i] = opaque(msc + 512u * (u32)a + 256u * (u32)i + 32u * (u32)k + 16u * (u32)(((g >> 1) ^ a) ^ i) +
                           8u * (u32)(g & 1));
          // Lane 16g + 8a + b writes group G = 8 (g ^ 2a) + b at p(G); a write
          // pass of 8 lanes (one g and a) covers 32 distinct banks.
          const int a2 = (lane >> 3) & 1, b = lane & 7;
          const int pg = ((2 * (g ^ (2 * a2)) + (b >> 2)) ^ (b & 2)) + 8 * (b & 3);
          tw = opaque(msc + 32u * (u32)pg + 16u * (u32)(a2 ^ (b & 1)));
        }
        sel = 0;
      } else {
        // MD 16 reads the row's 8 scale bytes of a stage and picks groups gi
        // and 4 + gi (byte 0x0c of a v_perm selector yields zero); MD 32 reads
        // the dword of groups 4gi..4gi+3 directly.  Fragment rows are multiples
        // of 16, so the row swap depends on rr only.
        const u32 word = G::MD == 32 ? 4u * gi : 0u;
        const int ssw = (rr >> 3) & 1;
#pragma unroll
        for (int g = 0; g < (G::NW == 4 ? 2 : 1); ++g) {
          bS[0][g] = opaque(lds0 + kScaleBase + (u32)(wm * G::FM * G::MD + rr) * kScRowBytes + 16 * (g ^ ssw) + word);
          bS[1][g] =
              opaque(lds0 + kScaleBase + (u32)(256 + wn * G::FN * G::MD + rr) * kScRowBytes + 16 * (g ^ ssw) + word);
        }
        sel = (u32)gi | ((u32)(4 + gi) << 8) | 0x0c0c0000u;
      }
    } else {
      sel = 0;
    }
  }

  G9_DEV rsrc_t src(int X) const { return X < 2 ? rA[X & 1] : rB[X & 1]; }
  // SGPR offset of stage `stage` in an operand row (kDeadOff past the end).
  G9_DEV u32 stage_off(int stage) const { return stage < s_end ? (u32)stage * kRowBytes : kDeadOff; }
  // SGPR offset of the chunk starting at stage `stage`: in a scale row, or
  // (FP4P) the chunk's offset in the scale array (stage is a multiple of 4).
  G9_DEV u32 chunk_off(int stage) const {
    if constexpr (I::kPreshuffled)
      return stage < s_end ? (u32)(stage / kScChunk) * cstride : kDeadOff;
    else if constexpr (I::kKMajor)
      return stage < s_end ? (u32)stage * 8 * cstride : kDeadOff;
    else
      return stage < s_end ? (u32)stage * 8 : kDeadOff;
  }

  // 16-byte DMA number J (rows 8J..8J+7 of the wave's kDmaRows) of sub-buffer X.
  // `mb` is mrow, passed through opaque_s once per region: the 8 distinct
  // LDS destinations (sub-buffer x slot) then cost one s_add per region
  // instead of SGPRs held for the whole loop; J moves the destination through
  // the immediate offset.
  template <int X, int SLOT, int J>
  G9_DEV void dma_rows(rsrc_t r, u32 soff, u32 mb) const {
    const u32 dst = mb + sub_off(X, SLOT);
    dma16<J * 1024>(r, (G9_LDS void*)(uintptr_t)dst, X < 2 ? vA[J] : vB[J], soff);
  }
  // Part J of the scale chunk whose rows start at `soff` bytes, into chunk slot SSLOT.
  template <int SSLOT, int J>
  G9_DEV void dma_chunk(u32 soff, u32 mb) const {
    if constexpr (I::kPreshuffled) {
      const u32 dst = mb + SSLOT * kScSlotBytes;
      dma16<J * 1024>(rS, (G9_LDS void*)(uintptr_t)dst, vS[0], soff);
    } else {
      const u32 dst = mb + SSLOT * kScSlotBytes + J * 1024;
      dma16(rS, (G9_LDS void*)(uintptr_t)dst, vS[J], soff);
    }
  }

  // 16-byte LDS read number R (fragment R / NC, chunk R % NC) of sub-buffer X.
  template <int X, int SLOT, int R>
  G9_DEV void read_chunk(FragSet<G>& f) const {
    constexpr int NC = G::NC;
    constexpr int region = X < 2 ? 0 : 65536;
    constexpr int imm = sub_off(X, SLOT) - region + (R / NC) * G::MD * kRowBytes;
    const u32 base = X < 2 ? bA[R % NC] : bB[R % NC];
    f[R / NC].c[R % NC] = *(const G9_LDS u32x4*)(uintptr_t)(base + imm);
  }
  // Scales of fragment F of sub-buffer X for stage ST of the chunk in slot SSLOT.
  template <int X, int SSLOT, int ST, int F>
  G9_DEV void read_scales(FragSet<G>& f) const {
    constexpr int imm = SSLOT * kScSlotBytes + (X & 1) * 128 * kScRowBytes + F * G::MD * kScRowBytes + 8 * (ST & 1);
    u32 base = bS[X >= 2][0];
    if constexpr (G::NW == 4) {
      base = bS[X >= 2][ST >> 1];
    } else if constexpr (ST >= 2) {
      // 8 waves have half the VGPRs: the stages 2-3 base differs from the
      // stages 0-1 base in address bit 4 only (the half swap), so it is formed
      // at the read (inline, so it is not hoisted into a loop-long register).
      asm volatile("v_xor_b32 %0, 16, %0" : "+v"(base));
    }
    if constexpr (G::MD == 16)
      f[F].sc = *(const G9_LDS u32x2*)(uintptr_t)(base + imm);
    else
      f[F].sp = *(const G9_LDS u32*)(uintptr_t)(base + imm);
  }

  // kChunkScales: the chunk's scales of fragment F of sub-buffer X from
  // chunk slot SSLOT (B0 into its registers of chunk parity PAR).
  template <int X, int SSLOT, int PAR, int F>
  G9_DEV void read_chunk_scales(ScRegs<OP, G>& sr) const {
    u32x2 v;
    if constexpr (I::kKMajor) {
      u32 base = bS[X >= 2][0];
      // Formed at the read (inline, so it is not hoisted into a loop-long
      // register).
      if constexpr (F != 0) asm volatile("v_xor_b32 %0, %1, %2" : "=v"(base) : "i"(16 * F), "v"(bS[X >= 2][0]));
      v = tr_read<SSLOT * kScSlotBytes + (X & 1) * 4096>(base);
    } else if constexpr (kTrScales<OP, G>) {
      v = tr_read<SSLOT * kScSlotBytes + (X & 1) * 4096 + (F / 2) * 1024>(bS[X >= 2][F & 1]);
    } else {
      constexpr int imm = SSLOT * kScSlotBytes + (X & 1) * 128 * kScRowBytes + F * G::MD * kScRowBytes;
      v = *(const G9_LDS u32x2*)(uintptr_t)(bS[X >= 2][0] + imm);
    }
    if constexpr (X == 0)
      sr.a[0][F] = v;
    else if constexpr (X == 1)
      sr.a[1][F] = v;
    else if constexpr (X == 2)
      sr.b0[PAR][F] = v;
    else
      sr.b1[F] = v;
  }

  // kXform: the two transpose reads of part J of this wave's rows in chunk
  // slot SSLOT, and (a region later, once they have landed) their writes.
  template <int SSLOT, int J>
  G9_DEV void xform_read(ScRegs<OP, G>& sr) const {
    constexpr int imm = SSLOT * kScSlotBytes + J * 1024;
    sr.t[0] = tr_read<imm>(tb[0]);
    sr.t[1] = tr_read<imm>(tb[1]);
  }
  template <int SSLOT, int J>
  G9_DEV void xform_write(const ScRegs<OP, G>& sr) const {
    lds_store16<SSLOT * kScSlotBytes + J * 1024>(tw, sr.t[0], sr.t[1]);
  }

  // Whole-set variants for the prologue.  Stage 0 of a K tail: the lanes
  // whose 16-byte chunk lies before k = 0 (chunk * 16 < kshift) get a dead
  // offset, so they load zeros instead of the previous row's last bytes (or
  // bytes before the operand).  Only the prologue ever issues stage 0.
  template <int X, int SLOT>
  G9_DEV void issue(int stage) const {
    const rsrc_t r = src(X);
    const u32 soff = stage_off(stage);
    if (stage == 0 && kshift != 0) {
      const int lane = fresh_tid_at(wave << 6) & 63;
      static_for<D>([&](auto J) {
        constexpr int j = decltype(J)::value;
        const int row = G::kDmaRows * wave + 8 * j + (lane >> 3);
        const int ch = (lane & 7) ^ ((row >> 1) & 7);
        const u32 v = (u32)ch * 16 < kshift ? kDeadOff : (X < 2 ? vA[j] : vB[j]);
        dma16<j * 1024>(r, (G9_LDS void*)(uintptr_t)(mrow + sub_off(X, SLOT)), v, soff);
      });
      return;
    }
    [&]<int... J>(std::integer_sequence<int, J...>) { (dma_rows<X, SLOT, J>(r, soff, mrow), ...); }(
        std::make_integer_sequence<int, D>{});
  }
  template <int SSLOT, int J>
  G9_DEV void issue_chunk(int stage) const {
    dma_chunk<SSLOT, J>(chunk_off(stage), msc);
  }
  template <int X, int SLOT, int SSLOT, int ST>
  G9_DEV void load(FragSet<G>& f) const {
    constexpr int NF = X < 2 ? G::FM : G::FN;
    [&]<int... R>(std::integer_sequence<int, R...>) { (read_chunk<X, SLOT, R>(f), ...); }(
        std::make_integer_sequence<int, G::NC * NF>{});
    if constexpr (I::kScaled && !kChunkScales<OP, G>) {
      [&]<int... F>(std::integer_sequence<int, F...>) { (read_scales<X, SSLOT, ST, F>(f), ...); }(
          std::make_integer_sequence<int, NF>{});
    }
  }
  // Packs fragment F's two scale bytes of each MFMA step into one register
  // (byte e = step e), so the MFMA selects its scale with op_sel.
  template <int X, int F>
  G9_DEV void gather_one(FragSet<G>& f) const {
    f[F].sp = __builtin_amdgcn_perm(f[F].sc.y, f[F].sc.x, sel);
  }
  template <int X>
  G9_DEV void gather_scales(FragSet<G>& f) const {
    constexpr int NF = X < 2 ? G::FM : G::FN;
    static_for<NF>([&](auto F) { gather_one<X, decltype(F)::value>(f); });
  }
};

// Per-quadrant accumulators of one wave.
template <class G>
using QAcc = accv<G>[G::FM][G::FN];
template <class G>
using Acc = accv<G>[2][2][G::FM][G::FN];

// Puts every accumulator in an AGPR at this point.  Called where a tile's
// accumulation starts, so the values the main loop's MFMAs tie to AGPRs
// arrive there from every path (zeroing or a stream-K partial) and the
// register allocator has no reason to stage them in VGPRs.
template <class G>
G9_DEV void pin_acc(Acc<G>& acc) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int j = 0; j < G::FN; ++j) asm volatile("" : "+a"(acc[q >> 1][q & 1][i][j]));
}

// Waits out the last MFMAs, then redefines every accumulator after the wait.
// Ends every path out of an MFMA stream: anything the compiler later
// generates to read the accumulators (copies at a control-flow join, spills,
// the epilogue) then reads the redefined values and so comes after the wait
// states, which it would not insert itself after inline-assembly MFMAs.
// isa_check.py verifies the built kernels for exactly this.
template <class G>
G9_DEV void settle_acc(Acc<G>& acc) {
  mfma_drain();
  pin_acc<G>(acc);
}

// Ends every path out of a stage sequence that issued inline-assembly scale
// reads (kTrScales): waits for them, then keeps their registers live up to
// that point, so the compiler neither reuses a register whose LDS read is
// still in flight (a read whose result a partial body never consumes is dead
// to it) nor touches one early.  isa_check.py verifies the built code.
template <Op OP, class G>
G9_DEV void settle_scales(ScRegs<OP, G>& sr) {
  if constexpr (kTrScales<OP, G>) {
    waitcnt<63, 0>();
    asm volatile("" : "+v"(sr.t[0]), "+v"(sr.t[1]));
#pragma unroll
    for (int i = 0; i < G::FM; ++i) asm volatile("" : "+v"(sr.a[0][i]), "+v"(sr.a[1][i]));
#pragma unroll
    for (int j = 0; j < G::FN; ++j) asm volatile("" : "+v"(sr.b1[j]), "+v"(sr.b0[0][j]), "+v"(sr.b0[1][j]));
  }
}

// Slot K of the region at body position POS: MFMA number K (step-major: step,
// A fragment, B fragment), then whatever the slot table puts after it, then a
// hard scheduling fence (the MFMAs are inline assembly, which the scheduler's
// instruction-class masks do not cover, so only a full fence pins the order).
// MFMA number K of the region at body position POS (step-major: step, A
// fragment, B fragment).  Snake order over the fragment grid: odd A fragments
// walk the B fragments backwards, so consecutive MFMAs share one operand
// register set.  The chip is power-limited in this loop and fewer operand
// changes cost less energy (measured: about 0.8% less time for every dtype,
// identical results).
template <Op OP, class G, int POS, int K>
G9_DEV void region_mfma(QAcc<G>& acc, const ScRegs<OP, G>& sr, const FragSet<G>& bx, const FragSet<G>& ay) {
  constexpr int e = K / (G::FM * G::FN), i = (K / G::FN) % G::FM, j0 = K % G::FN;
  constexpr int j = (i % 2) ? G::FN - 1 - j0 : j0;
  if constexpr (kChunkScales<OP, G>) {
    // Region POS % 4 is quadrant (A0,B0), (A0,B1), (A1,B1), (A1,B0); its
    // stage is stage POS / 4 % 4 of chunk POS / 16 of the body.
    constexpr int quad = POS % 4, st = (POS / 4) % kScChunk, cp = (POS / 16) % 2;
    const u32x2& sa = sr.a[quad >= 2 ? 1 : 0][i];
    const u32x2& sb = (quad == 1 || quad == 2) ? sr.b1[j] : sr.b0[cp][j];
    mfma_scaled<2 * (st & 1) + e>(acc[i][j], bx[j].c[e], ay[i].c[e], (st >> 1) ? sb.y : sb.x,
                                  (st >> 1) ? sa.y : sa.x);
  } else {
    mma<OP, G, e>(acc[i][j], bx[j], ay[i]);
  }
}

template <Op OP, class G, int RX, int RSLOT, int DX, int DSLOT, int POS, int K>
G9_DEV void region_slot(const Pipe<OP, G>& P, rsrc_t r, u32 soff, u32 soff_sc, u32 mb, u32 ms, QAcc<G>& acc,
                        ScRegs<OP, G>& sr, const FragSet<G>& bx, const FragSet<G>& ay, FragSet<G>& nxt) {
  constexpr int NF = RX < 2 ? G::FM : G::FN;
  using S = Slots<OP, G, NF>;
  using Sh = Shape<OP, G>;
  // The stage (in the body) whose operands this region reads: the current one
  // in regions 0-1, the next one in regions 2-3; its scale chunk slot and
  // stage within the chunk.
  constexpr int ks = POS / 4 + (POS % 4 >= 2 ? 1 : 0);
  constexpr int kSSlot = (ks / kScChunk) % 2, kSt = ks % kScChunk;
  // Scale-chunk DMA of this position: part 0 goes to the chunk two ahead of
  // the current one (the current chunk's slot, free since position 16h + 13),
  // the other parts to the next chunk's slot.
  constexpr int part = Sh::sc_part(POS);
  constexpr int kDSSlot = part == 0 ? (POS / 16) % 2 : (POS / 16 + 1) % 2;
  region_mfma<OP, G, POS, K>(acc, sr, bx, ay);
  constexpr int q = K - S::kPre;
  if constexpr (q >= 0) {
    static_for<S::NR>([&](auto R) {
      if constexpr (S::read_q(decltype(R)::value) == q) P.template read_chunk<RX, RSLOT, decltype(R)::value>(nxt);
    });
    if constexpr (kChunkScales<OP, G>) {
      // The chunk's scales of set RX, when RX is read for a chunk's first stage.
      if constexpr (kSt == 0) {
        static_for<NF>([&](auto F) {
          if constexpr (S::scale_q(decltype(F)::value) == q)
            P.template read_chunk_scales<RX, kSSlot, (ks / kScChunk) % 2, decltype(F)::value>(sr);
        });
      }
    } else if constexpr (OpInfo<OP>::kScaled) {
      static_for<NF>([&](auto F) {
        if constexpr (S::scale_q(decltype(F)::value) == q)
          P.template read_scales<RX, kSSlot, kSt, decltype(F)::value>(nxt);
      });
    }
    static_for<S::D>([&](auto J) {
      if constexpr (S::dma_q(decltype(J)::value) == q) P.template dma_rows<DX, DSLOT, decltype(J)::value>(r, soff, mb);
    });
    if constexpr (part >= 0 && q == S::kScaleDmaQ) P.template dma_chunk<kDSSlot, (part >= 0 ? part : 0)>(soff_sc, ms);
    if constexpr (kXform<OP, G>) {
      // Transpose of the next chunk (slot xs): part j is read at body
      // position 16h + R(j), R = 5, 8, 10, 12 -- at least 7 regions after its
      // DMA (16h - 2 + 2j), which the region-start vmcnt wait has completed
      // -- and written one region later, in the same stage, so a partial
      // body never stops between the two.  The last writes land before the
      // barrier of position 16h + 14, whose region first reads the chunk.
      constexpr int p16 = POS % 16, xs = (POS / 16 + 1) % 2;
      constexpr int rj = p16 == 5 ? 0 : p16 == 8 ? 1 : p16 == 10 ? 2 : p16 == 12 ? 3 : -1;
      constexpr int wj = p16 == 6 ? 0 : p16 == 9 ? 1 : p16 == 11 ? 2 : p16 == 13 ? 3 : -1;
      if constexpr (rj >= 0 && q == S::kXformQ) P.template xform_read<xs, (rj >= 0 ? rj : 0)>(sr);
      if constexpr (wj >= 0 && q == S::kXformQ) P.template xform_write<xs, (wj >= 0 ? wj : 0)>(sr);
    }
    if constexpr (OpInfo<OP>::kScaled && !kChunkScales<OP, G> && G::MD == 16) {
      static_for<NF>([&](auto F) {
        constexpr int f = decltype(F)::value;
        if constexpr (S::perm_q(f) == q) {
          if constexpr (f == 0) waitcnt<63, 0>();  // the region's scale reads landed
          P.template gather_one<RX, f>(nxt);
        }
      });
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

#ifndef G9_PINGPONG
#define G9_PINGPONG 1
#endif
// 8-wave kernels run the ping-pong schedule below.
template <class G>
constexpr bool kPingPong = G9_PINGPONG != 0 && G::NW == 8;
#ifndef G9_HALF_BARRIER
#define G9_HALF_BARRIER 1
#endif
// The other FP16, BF16 and MXFP4 kernels pass a barrier at even body
// positions only (see stage()): measured interleaved on two boxes against a
// barrier in every region, 0.8-1.0% less time for FP16, 0.4-1.3% for BF16,
// 0.5-1.2% for MXFP4 (all three scale layouts), results identical.  BF8's
// regions are twice as long (32-cycle MFMAs) and it measured no faster, so it
// keeps a barrier per region.
template <Op OP, class G>
constexpr bool kHalfBarrier = G9_HALF_BARRIER != 0 && !kPingPong<G> && OP != Op::BF8;

// The quadrant region at body position POS (region POS % 4 of stage s + POS / 4,
// with s the body's first stage): MFMAs of (bx, ay) into acc, LDS reads of
// sub-buffer RX/RSLOT into nxt, DMA of stage `ds` into sub-buffer DX/DSLOT.
//   s_waitcnt vmcnt(DMAs of the 6 previous regions) lgkmcnt(0)
//                                          -- DMA of the set read now landed,
//                                             the previous region's reads done
//   kPre MFMAs
//   s_barrier                              -- every wave's DMA landed and every
//                                             wave done reading the sub-buffer
//                                             refilled now
//   remaining MFMAs with the reads and DMAs interleaved
// kHalfBarrier: odd positions wait for the previous region's reads only and
// pass no barrier (their MFMAs, reads and DMAs in the same slots); even
// positions wait for the DMAs of 5 regions earlier (vm_wait_hb).
template <Op OP, class G, int RX, int RSLOT, int DX, int DSLOT, int POS>
G9_DEV void region(const Pipe<OP, G>& P, int s, int ds, QAcc<G>& acc, ScRegs<OP, G>& sr, const FragSet<G>& bx,
                   const FragSet<G>& ay, FragSet<G>& nxt) {
  constexpr int NF = RX < 2 ? G::FM : G::FN;
  using S = Slots<OP, G, NF>;
  using Sh = Shape<OP, G>;
  constexpr bool kBar = !kHalfBarrier<OP, G> || POS % 2 == 0;
  constexpr int kVm = !kHalfBarrier<OP, G> ? Sh::vm_wait(POS) : kBar ? Sh::vm_wait_hb(POS) : 63;
  __builtin_amdgcn_sched_barrier(0);
  waitcnt<kVm, 0>();
  const rsrc_t r = P.src(DX);
  const u32 soff = P.stage_off(ds);
  const u32 mb = opaque_s(P.mrow);
  u32 soff_sc = 0, ms = 0;
  if constexpr (Sh::sc_part(POS) >= 0) {
    soff_sc = P.chunk_off(s + kScChunk * (POS / 16) + (Sh::sc_part(POS) == 0 ? 2 : 1) * kScChunk);
    ms = opaque_s(P.msc);
  }
  [&]<int... K>(std::integer_sequence<int, K...>) {
    (region_slot<OP, G, RX, RSLOT, DX, DSLOT, POS, K>(P, r, soff, soff_sc, mb, ms, acc, sr, bx, ay, nxt), ...);
  }(std::make_integer_sequence<int, S::kPre>{});
  if constexpr (kBar) barrier();
  [&]<int... K>(std::integer_sequence<int, K...>) {
    (region_slot<OP, G, RX, RSLOT, DX, DSLOT, POS, K + S::kPre>(P, r, soff, soff_sc, mb, ms, acc, sr, bx, ay, nxt),
     ...);
  }(std::make_integer_sequence<int, S::NM - S::kPre>{});
}

// ---------------------------------------------------------------------------
// 8-wave ping-pong.  The two waves of a SIMD (waves w and w + 4) run the same
// region sequence one cluster apart: each region is split into an MFMA
// cluster (its MFMAs only, at wave priority 0) and a memory cluster (the next
// region's LDS reads and this region's DMAs, at priority 1), with a workgroup
// barrier at every cluster boundary.  Waves 4-7 take one extra barrier before
// the loop, so whenever waves 0-3 run an MFMA cluster waves 4-7 run a memory
// cluster and the other way round: one wave of each SIMD keeps the matrix
// unit busy while the other issues its reads and DMAs beside it, and the
// memory cluster's higher priority lets it issue in the MFMA stream's free
// slots.  Waves 0-3 take the matching extra barrier after the loop.
//
// Ordering, with groups a cluster apart:
//  * a memory cluster ends with lgkmcnt(0) before its barrier, so its reads
//    have landed before any wave passes the barrier -- the next MFMA cluster's
//    operands, and the sub-buffer they came from is free for the DMA the next
//    memory cluster issues (the other group's reads of it ended one barrier
//    earlier);
//  * a memory cluster also waits, before its barrier, for its DMAs of 6
//    regions earlier: the next memory cluster of the leading group reads them
//    after that barrier.  The lagging group waits one region earlier than its
//    own reads need, so the DMA lead is 6 regions instead of 7.
// ---------------------------------------------------------------------------
template <Op OP, class G, int RX, int RSLOT, int DX, int DSLOT, int POS>
G9_DEV void region_pp(const Pipe<OP, G>& P, int s, int ds, QAcc<G>& acc, ScRegs<OP, G>& sr, const FragSet<G>& bx,
                      const FragSet<G>& ay, FragSet<G>& nxt) {
  constexpr int NF = RX < 2 ? G::FM : G::FN;
  using Sh = Shape<OP, G>;
  static_assert(!kChunkScales<OP, G>, "chunk-wide scale reads run 4-wave");
  constexpr int ks = POS / 4 + (POS % 4 >= 2 ? 1 : 0);
  constexpr int kSSlot = (ks / kScChunk) % 2, kSt = ks % kScChunk;
  constexpr int part = Sh::sc_part(POS);
  constexpr int kDSSlot = part == 0 ? (POS / 16) % 2 : (POS / 16 + 1) % 2;
  // MFMA cluster.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(0);
  static_for<Sh::NM>([&](auto K) {
    region_mfma<OP, G, POS, decltype(K)::value>(acc, sr, bx, ay);
    __builtin_amdgcn_sched_barrier(0);
  });
  barrier();
  // Memory cluster.
  __builtin_amdgcn_s_setprio(1);
  const rsrc_t r = P.src(DX);
  const u32 soff = P.stage_off(ds);
  const u32 mb = opaque_s(P.mrow);
  static_for<G::NC * NF>([&](auto R) { P.template read_chunk<RX, RSLOT, decltype(R)::value>(nxt); });
  if constexpr (OpInfo<OP>::kScaled)
    static_for<NF>([&](auto F) { P.template read_scales<RX, kSSlot, kSt, decltype(F)::value>(nxt); });
  static_for<Sh::D>([&](auto J) { P.template dma_rows<DX, DSLOT, decltype(J)::value>(r, soff, mb); });
  if constexpr (part >= 0) {
    const u32 soff_sc = P.chunk_off(s + kScChunk * (POS / 16) + (part == 0 ? 2 : 1) * kScChunk);
    P.template dma_chunk<kDSSlot, (part >= 0 ? part : 0)>(soff_sc, opaque_s(P.msc));
  }
  if constexpr (OpInfo<OP>::kScaled && G::MD == 16) {
    waitcnt<63, 0>();
    P.template gather_scales<RX>(nxt);
  }
  waitcnt<Sh::vm_wait_pp(POS), 0>();
  barrier();
}

// Stage K of the body starting at stage s.  Even stages (operand slot 0): B0
// fragments in x; B1 fragments go to y, and after they are consumed the next
// stage's B0 fragments go to y as well.  Odd stages (slot 1): B0 in y; B1 to
// x, then the next stage's B0.
//
// Each region reads one sub-buffer (B1, A1, then the next stage's A0 and B0)
// and refills one that every wave has finished reading, i.e. one read before
// the last barrier.  With a barrier in every region that is the sub-buffer
// read in the previous region (the last region refills the next stage's A0
// with stage + 3).  kHalfBarrier: an odd region's last barrier is its
// predecessor's, so every region refills the sub-buffer read two regions
// earlier: stage K's four regions refill A0, B0, B1, A1 of its slot with stage
// K + 2, the prologue's order.  Each sub-buffer is read again 6 regions after
// its refill, at an even position or right after one; the even region's wait
// (vm_wait_hb) covers both.
template <Op OP, class G, int K>
G9_DEV void stage(const Pipe<OP, G>& P, int s, Acc<G>& acc, ScRegs<OP, G>& sr, FragSet<G>& at, FragSet<G>& ab,
                  FragSet<G>& x, FragSet<G>& y) {
  constexpr int POS = 4 * K;
  auto rg = [&]<int RX, int RSLOT, int DX, int DSLOT, int P_>(int ds, QAcc<G>& a, const FragSet<G>& bx,
                                                                const FragSet<G>& ay, FragSet<G>& nxt) {
    if constexpr (kPingPong<G>)
      region_pp<OP, G, RX, RSLOT, DX, DSLOT, P_>(P, s, ds, a, sr, bx, ay, nxt);
    else
      region<OP, G, RX, RSLOT, DX, DSLOT, P_>(P, s, ds, a, sr, bx, ay, nxt);
  };
  if constexpr (kHalfBarrier<OP, G>) {
    constexpr int sl = K % 2, nx = 1 - sl;
    FragSet<G>& b0 = sl ? y : x;  // this stage's B0 fragments
    FragSet<G>& b1 = sl ? x : y;  // its B1, then the next stage's B0
    rg.template operator()<3, sl, 0, sl, POS + 0>(s + K + 2, acc[0][0], b0, at, b1);
    rg.template operator()<1, sl, 2, sl, POS + 1>(s + K + 2, acc[0][1], b1, at, ab);
    rg.template operator()<0, nx, 3, sl, POS + 2>(s + K + 2, acc[1][1], b1, ab, at);
    rg.template operator()<2, nx, 1, sl, POS + 3>(s + K + 2, acc[1][0], b0, ab, b1);
  } else if constexpr (K % 2 == 0) {
    rg.template operator()<3, 0, 2, 0, POS + 0>(s + K + 2, acc[0][0], x, at, y);
    rg.template operator()<1, 0, 3, 0, POS + 1>(s + K + 2, acc[0][1], y, at, ab);
    rg.template operator()<0, 1, 1, 0, POS + 2>(s + K + 2, acc[1][1], y, ab, at);
    rg.template operator()<2, 1, 0, 1, POS + 3>(s + K + 3, acc[1][0], x, ab, y);
  } else {
    rg.template operator()<3, 1, 2, 1, POS + 0>(s + K + 2, acc[0][0], y, at, x);
    rg.template operator()<1, 1, 3, 1, POS + 1>(s + K + 2, acc[0][1], x, at, ab);
    rg.template operator()<0, 0, 1, 1, POS + 2>(s + K + 2, acc[1][1], x, ab, at);
    rg.template operator()<2, 0, 0, 0, POS + 3>(s + K + 3, acc[1][0], y, ab, x);
  }
}

// The last n < kBody stages (a partial body): stages 0 .. n-1.
template <Op OP, class G, int K>
G9_DEV void tail(const Pipe<OP, G>& P, int s, int n, Acc<G>& acc, ScRegs<OP, G>& sr, FragSet<G>& at, FragSet<G>& ab,
                 FragSet<G>& x, FragSet<G>& y) {
  if constexpr (K + 1 < Shape<OP, G>::kBody) {
    if (n > K) {
      stage<OP, G, K>(P, s, acc, sr, at, ab, x, y);
      tail<OP, G, K + 1>(P, s, n, acc, sr, at, ab, x, y);
    }
  }
}

// Accumulates stages [s0, s1) of tile (tm, tn) into acc.  Leaves every DMA
// complete and the workgroup synchronised, so LDS is free on return.
template <Op OP, class G>
G9_DEV void mainloop(const GemmParams& p, char* smem, int tm, int tn, int s0, int s1, Acc<G>& acc,
                     bool stamp = false, int wb = -1) {
  using Sh = Shape<OP, G>;
  constexpr bool kScaled = OpInfo<OP>::kScaled;
  Pipe<OP, G> P;
  P.init(p, smem, tm, tn, s0, s1, wb);
  // Scale chunk 0 (stages s0 .. s0+3) first, then the operands in DMA stream
  // order, per stage A0, B0, B1, A1 (stage s lives in slot (s-s0)&1), with
  // part 0 of chunk 1 where body position 30 would issue it: the prologue
  // then leaves the DMA counts the first body's waits expect.
  if constexpr (kScaled) static_for<G::kScParts>([&](auto J) { P.template issue_chunk<0, decltype(J)::value>(s0); });
  P.template issue<0, 0>(s0);
  P.template issue<2, 0>(s0);
  P.template issue<3, 0>(s0);
  P.template issue<1, 0>(s0);
  P.template issue<0, 1>(s0 + 1);
  P.template issue<2, 1>(s0 + 1);
  P.template issue<3, 1>(s0 + 1);
  P.template issue<1, 1>(s0 + 1);
  if constexpr (kScaled) P.template issue_chunk<1, 0>(s0 + kScChunk);
  // A0(s0) and B0(s0) landed (and chunk 0, issued before them): read them,
  // then (once every wave has) refill A0 slot 0 with stage s0+2.  Ping-pong:
  // B1(s0) as well, which the first memory cluster reads.
  constexpr int kFirst = (kPingPong<G> ? 5 : 6) * Sh::D + (kScaled ? 1 : 0);
  ScRegs<OP, G> sr;
  waitcnt<kFirst, 0>();
  if constexpr (kXform<OP, G>) {
    // This wave's parts of chunk 0 have landed: transpose them before any
    // wave reads the chunk (the barrier below), all reads first (one LDS
    // round trip for the chunk, in registers the loop has not claimed yet).
    ScRegs<OP, G> xs[G::kScParts];
    static_for<G::kScParts>([&](auto J) { P.template xform_read<0, decltype(J)::value>(xs[J]); });
    waitcnt<63, 0>();
    static_for<G::kScParts>([&](auto J) { P.template xform_write<0, decltype(J)::value>(xs[J]); });
    waitcnt<63, 0>();
  }
  barrier();
  FragSet<G> at, ab, x, y;
  P.template load<0, 0, 0, 0>(at);
  P.template load<2, 0, 0, 0>(x);
  if constexpr (kChunkScales<OP, G>) {
    // Chunk 0's scales of A0 and B0 (read by body positions -2 and -1 in the
    // steady state); B1's and A1's follow in the first two regions.
    static_for<G::FM>([&](auto F) { P.template read_chunk_scales<0, 0, 0, decltype(F)::value>(sr); });
    static_for<G::FN>([&](auto F) { P.template read_chunk_scales<2, 0, 0, decltype(F)::value>(sr); });
  }
  waitcnt<kFirst, 0>();
  if constexpr (kScaled && !kChunkScales<OP, G> && G::MD == 16) {
    P.template gather_scales<0>(at);
    P.template gather_scales<2>(x);
  }
  barrier();
  // The refill of A0's slot 0 the region before the loop would issue (with a
  // barrier per region; kHalfBarrier: the loop's first region issues it).
  if constexpr (!kHalfBarrier<OP, G>) P.template issue<0, 0>(s0 + 2);
  // Ping-pong: waves 4-7 start one cluster behind.
  const bool lag = kPingPong<G> && P.wave >= 4;
  if (lag) barrier();
  // The accumulators were just written by VALU (zeroing or a partial tile):
  // wait states before the first MFMA reads them.
  mfma_drain();
  // kBody stages per iteration (the B registers swap roles between stages),
  // then the remaining stages as a partial body.
  if (stamp) timing_stamp(1);
  int s = s0;
  for (; s + Sh::kBody <= s1; s += Sh::kBody)
    static_for<Sh::kBody>([&](auto K) { stage<OP, G, decltype(K)::value>(P, s, acc, sr, at, ab, x, y); });
  settle_scales<OP, G>(sr);
  settle_acc<G>(acc);
  if (s < s1) {
    tail<OP, G, 0>(P, s, s1 - s, acc, sr, at, ab, x, y);
    settle_scales<OP, G>(sr);
    settle_acc<G>(acc);
  }
  if constexpr (kPingPong<G>) {
    // Waves 0-3 match the lagging group's last barrier; back to priority 0.
    if (!lag) barrier();
    __builtin_amdgcn_s_setprio(0);
  }
  waitcnt<0, 0>();
  barrier();
}

template <class G>
G9_DEV void zero_acc(Acc<G>& acc) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int j = 0; j < G::FN; ++j) acc[q >> 1][q & 1][i][j] = accv<G>{};
}

// Eight 16-bit outputs of row m from column col on: one non-temporal 16-byte
// store (C streams out without displacing the A/B blocks the XCD's other
// workgroups still read from L2; measured, interleaved: 1.4% less time for
// FP16, 1.1% BF16, 0.4% BF8, 2.5% MXFP4), or element stores masked at N.
G9_DEV void put_c16(const GemmParams& p, int m, int col, u32x4 d) {
  if (m >= p.M) return;
  char* dst = p.c + ((size_t)m * p.ldc + col) * 2;
  if (col + 8 <= p.N && ((uintptr_t)dst & 15) == 0) {
    __builtin_nontemporal_store(d, reinterpret_cast<u32x4*>(dst));
  } else {
    const uint16_t* hv = reinterpret_cast<const uint16_t*>(&d);
    for (int e = 0; e < 8; ++e)
      if (col + e < p.N) reinterpret_cast<uint16_t*>(dst)[e] = hv[e];
  }
}

// Converts the tile to 16-bit (after multiplying by `scale`), stages it in LDS
// and writes it to C with coalesced, non-temporal 16-byte row chunks, masking
// rows >= M and columns >= N.  LDS must be free on entry; it is free again on
// return.
//
// The conversion (four AGPR reads, two packs and an LDS write per fragment) is
// VALU-bound, ~2.5k cycles for the whole tile at one wave per SIMD, and the
// stores cannot start before a row is staged.  So with 4 waves the tile goes
// out by quadrant: quadrant 0 is staged first, and the stores of each
// quadrant are issued interleaved with the conversion of the next one
// (distinct staging rows and columns), a barrier between quadrants.
//
// Staging layout: row m of the tile at m * 528 bytes, rows 16-byte aligned so
// the 16-byte reads stay aligned.  Measured on gfx950 (SQ_LDS_BANK_CONFLICT of
// probe kernels), a 64-lane ds_write_b64 is served 16 consecutive lanes at a
// time over 32 banks, so a write pass (16 rows of one 8-byte unit) sees the
// rows' 4-bank offsets wrap after 8 rows: 4 conflict cycles per write, 1024
// per workgroup.  A conflict-free variant (8-byte units XOR-swizzled by row,
// read back as swapped 16-byte pairs) measured 0 conflicts but 0.5-1.0% more
// time for every type, interleaved in one process: the epilogue is bound by
// the C write to HBM, and its extra address and swap instructions lengthened
// it by ~1.5k cycles.
template <int OUT, class G>
G9_DEV void store_tile(const GemmParams& p, char* smem, int tm, int tn, Acc<G>& acc, float scale, int wb = -1) {
  const int tid = fresh_tid(wb), lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WN, wn = wave % G::WN;
  const int rr = lane % G::MD, gi = lane / G::MD;
  // Fragment F = (i, j) of quadrant Q = (qm, qn), converted into its staging
  // rows.
  auto stage_frag = [&]<int Q, int F>() {
    constexpr int qm = Q >> 1, qn = Q & 1, i = F / G::FN, j = F % G::FN;
    // The fragment is copied to VGPRs here, where it is converted: without
    // the fence the compiler copies the whole tile to VGPRs ahead of any
    // branch leading here (stream-K: before choosing between this and the
    // partial store), where the copies outgrow the registers and spill.
    accv<G> f = acc[qm][qn][i][j];
    asm volatile("" : "+v"(f));
    static_for<G::NB>([&](auto B) {
      constexpr int b = decltype(B)::value;
      const int m = qm * 128 + wm * G::FM * G::MD + i * G::MD + rr;
      const int n = qn * 128 + wn * G::FN * G::MD + j * G::MD + 4 * G::NG * b + 4 * gi;
      const f32x4 v = get_quad<b>(f) * scale;
      const u32x2 h = OUT == OUT_BF16 ? pack4_bf16(v) : pack4_f16(v);
      lds_write8(smem + m * kStageRow + n * 2, h);
    });
  };
  constexpr int kFrags = G::FM * G::FN;             // fragments per quadrant
  constexpr int kRowsPerPass = G::kThreads / 16;    // 16 chunks of 16 bytes per quadrant row
  constexpr int kPasses = 128 / kRowsPerPass;       // store passes per quadrant
  const int ch = tid & 15;
  // Pass P of quadrant Q: row P * kRowsPerPass + tid / 16 of the quadrant.
  auto store_pass = [&]<int Q>(int pass) {
    constexpr int qm = Q >> 1, qn = Q & 1;
    const int r = qm * 128 + pass * kRowsPerPass + (tid >> 4);
    const int col = tn * kTile + qn * 128 + ch * 8;
    put_c16(p, tm * kTile + r, col, lds_read16(smem + r * kStageRow + (qn * 128 + ch * 8) * 2));
  };
  if constexpr (G::NW == 8) {
    // Two waves per SIMD: one converts while the other stores, so the tile
    // is staged whole and goes out in passes of whole 512-byte rows (the
    // quadrant variants measured 0.2-0.6% slower here).
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j) {
          accv<G> f = acc[q >> 1][q & 1][i][j];
          asm volatile("" : "+v"(f));
          static_for<G::NB>([&](auto B) {
            constexpr int b = decltype(B)::value;
            const int m = (q >> 1) * 128 + wm * G::FM * G::MD + i * G::MD + rr;
            const int n = (q & 1) * 128 + wn * G::FN * G::MD + j * G::MD + 4 * G::NG * b + 4 * gi;
            const f32x4 v = get_quad<b>(f) * scale;
            const u32x2 h = OUT == OUT_BF16 ? pack4_bf16(v) : pack4_f16(v);
            lds_write8(smem + m * kStageRow + n * 2, h);
          });
        }
    waitcnt<0, 0>();
    barrier();
    constexpr int kRows = G::kThreads / 32;
    const int c32 = tid & 31;
    const int col = tn * kTile + c32 * 8;
#pragma unroll 4
    for (int pass = 0; pass < kTile / kRows; ++pass) {
      const int r = pass * kRows + (tid >> 5);
      put_c16(p, tm * kTile + r, col, lds_read16(smem + r * kStageRow + c32 * 16));
    }
    barrier();
    return;
  }
  static_for<kFrags>([&](auto F) { stage_frag.template operator()<0, decltype(F)::value>(); });
  waitcnt<63, 0>();
  barrier();
  // Pass P of quadrant Q after the fragments F of quadrant Q + 1 with
  // F * kPasses / kFrags == P.
  static_for<3>([&](auto QC) {
    constexpr int Q = decltype(QC)::value;
    static_for<kPasses>([&](auto P) {
      constexpr int pass = decltype(P)::value;
      static_for<kFrags>([&](auto F) {
        constexpr int f = decltype(F)::value;
        if constexpr (f * kPasses / kFrags == pass) stage_frag.template operator()<Q + 1, f>();
      });
      store_pass.template operator()<Q>(pass);
      __builtin_amdgcn_sched_barrier(0);
    });
    waitcnt<63, 0>();
    barrier();
  });
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) store_pass.template operator()<3>(pass);
  barrier();
}

template <Op OP>
G9_DEV float epilogue_scale(const GemmParams& p) {
  if constexpr (OP == Op::BF8) {
    float s = 1.f;
    if (p.a_scale) s *= *p.a_scale;
    if (p.b_scale) s *= *p.b_scale;
    return s;
  } else {
    return 1.f;
  }
}

// Data-parallel schedule: one workgroup per 256x256 output tile.
template <Op OP, int OUT, class G>
G9_DEV void gemm_dp(const GemmParams& p) {
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes<OpInfo<OP>::kScaled>];
  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, p.num_xcds, p.group_m, tm, tn);
  Acc<G> acc;
  timing_stamp(0);
  zero_acc<G>(acc);
  pin_acc<G>(acc);
  mainloop<OP, G>(p, smem, tm, tn, 0, p.ns, acc, true);
  timing_stamp(2);
  store_tile<OUT, G>(p, smem, tm, tn, acc, epilogue_scale<OP>(p));
  timing_stamp(3);
}

// Grouped ("MoE") GEMM over E experts: expert e multiplies rows
// [off[e], off[e+1]) of A (tokens sorted by expert) by its own B_e (for BF8
// with its own fp32 scale b_scale[e]) into the same rows of C.  The grid covers tiles_m x tiles_n tiles with tiles_m an
// upper bound of the experts' m-tiles (sum of ceil(M_e / 256) <= ceil(M / 256)
// + E); each workgroup finds the expert of its m-tile and then runs the
// data-parallel tile unchanged on that expert's rows and weights.  Workgroups
// past the last expert's tiles exit.  Offsets are clamped to [0, M] (and each
// expert's end to at least its start), so any offset table keeps every access
// inside A, C and the experts' B.

// Expert of m-tile `mt`: 64 experts per pass, one per lane (their m-tile
// counts, an inclusive wave prefix sum, a ballot for the lane whose range
// holds mt).  Returns false if mt is past the last expert's tiles.
G9_DEV bool moe_find(const GemmParams& p, int mt, int& expert, int& local_mt, int& row0, int& rows) {
  const int lane = threadIdx.x & 63;
  const int T = p.M;
  int base = 0;
  for (int e0 = 0; e0 < p.moe_experts; e0 += 64) {
    const int e = e0 + lane;
    int lo = 0, hi = 0, n = 0;
    if (e < p.moe_experts) {
      lo = min(max(p.moe_off[e], 0), T);
      hi = min(max(p.moe_off[e + 1], lo), T);
      n = (hi - lo + kTile - 1) / kTile;
    }
    int incl = n;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    const int first = base + incl - n;
    const unsigned long long hit = __ballot(n > 0 && mt >= first && mt < base + incl);
    if (hit) {
      const int l = __ffsll((long long)hit) - 1;
      expert = __builtin_amdgcn_readfirstlane(__shfl(e, l, 64));
      local_mt = __builtin_amdgcn_readfirstlane(mt - __shfl(first, l, 64));
      row0 = __builtin_amdgcn_readfirstlane(__shfl(lo, l, 64));
      rows = __builtin_amdgcn_readfirstlane(__shfl(hi - lo, l, 64));
      return true;
    }
    base += __shfl(incl, 63, 64);
  }
  return false;
}

template <Op OP, int OUT, class G>
G9_DEV void gemm_moe(const GemmParams& p) {
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes<OpInfo<OP>::kScaled>];
  int mt, tn;
  tile_coords(blockIdx.x, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, p.num_xcds, p.group_m, mt, tn);
  int expert, tm, row0, rows;
  if (!moe_find(p, mt, expert, tm, row0, rows)) return;
  GemmParams q = p;
  q.a = p.a + (size_t)row0 * p.lda;
  q.c = p.c + (size_t)row0 * p.ldc * 2;
  q.b = p.b + (size_t)expert * p.moe_b_stride;
  q.M = rows;
  if constexpr (OpInfo<OP>::kScaled) {
    q.a_sc = p.a_sc + (size_t)row0 * p.ldsa;
    q.b_sc = p.b_sc + (size_t)expert * p.moe_bsc_stride;
  }
  if constexpr (OP == Op::BF8) {
    // BF8: one fp32 scale per expert for B (b_scale[expert]); A's is per tensor.
    if (p.b_scale) q.b_scale = p.b_scale + expert;
  }
  Acc<G> acc;
  zero_acc<G>(acc);
  pin_acc<G>(acc);
  mainloop<OP, G>(q, smem, tm, tn, 0, q.ns, acc, false);
  store_tile<OUT, G>(q, smem, tm, tn, acc, epilogue_scale<OP>(q));
}

// ---------------------------------------------------------------------------
// Stream-K schedule.
//
// The (tile, stage) space is linearised tile-major and cut into `sk_ctas`
// contiguous ranges, one per persistent workgroup.  A tile whose stages span
// several ranges is finished by a K-ordered chain: the owner of stages
// [sb, se) with sb > 0 waits for the tile's flag to read (epoch, sb), loads the
// predecessor's fp32 partial as its initial accumulator and continues, so
// every output element sees exactly the MFMA sequence of the data-parallel
// kernel and the result is bit-identical to it.  Each workgroup walks its
// range from the last tile backwards, so the prefix it owes a successor is
// produced first and the suffix it inherits is consumed last.
// ---------------------------------------------------------------------------

// Index (in f32x4) of a wave's fragment in a tile's partial: the accumulator
// register layout, so each wave access is a contiguous KiB.
template <class G>
G9_DEV int ws_index(int wave, int q, int i, int j, int b, int lane) {
  return (((wave * (4 * G::FM * G::FN) + (q * G::FM + i) * G::FN + j) * G::NB + b) * 64 + lane);
}

// The flag is read once per wave (readfirstlane), so the loop and everything
// after it stay wave-uniform in the compiler's eyes; a per-lane exit condition
// would make the buffer resources built after it look divergent.
G9_DEV void wait_flag(const GemmParams& p, int tile, u32 want) {
  u32 spins = 0;
  while (__builtin_amdgcn_readfirstlane(
             __hip_atomic_load(p.flags + tile, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) != want) {
    __builtin_amdgcn_s_sleep(2);
    if (++spins > p.spin_limit) {
      __hip_atomic_store(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // The host flag of g9_workspace_watch (a device-writable host int, or
      // null), so the caller sees the failure without synchronising.
      int* host = *reinterpret_cast<int* const*>(reinterpret_cast<const char*>(p.err) + 8);
      if (host) __hip_atomic_store(host, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      break;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

template <Op OP, int OUT, class G>
G9_DEV void sk_segment(const GemmParams& p, char* smem, int tile, int sb, int se, SkTimes& times, int wb) {
  // wb is lane 0's threadIdx.x, so the fallback of fresh_tid (which would
  // keep the raw index register alive through the persistent loop) is dead.
  __builtin_assume(wb >= 0);
  int tm, tn;
  // The grid sizes pass through opaque_s so the divisions are redone per
  // segment rather than their reciprocals held (in VGPRs) across the loop.
  const int tiles_m = (int)opaque_s((u32)p.tiles_m), tiles_n = (int)opaque_s((u32)p.tiles_n);
  tile_coords(tile, tiles_m * tiles_n, tiles_m, tiles_n, 1, (int)opaque_s((u32)p.group_m), tm, tn);
  // The thread index is formed separately before and after the main loop
  // (fresh_tid), so no VGPR holds it across the loop.
  f32x4* ws = reinterpret_cast<f32x4*>(p.ws) + (size_t)tile * (kTile * kTile / 4);
  Acc<G> acc;
  if (sb == 0) {
    zero_acc<G>(acc);
  } else {
    const int tid = fresh_tid(wb), lane = tid & 63, wave = tid >> 6;
    [[maybe_unused]] const unsigned long long t0 = clk();
    wait_flag(p, tile, (p.epoch << 16) | (u32)sb);
    [[maybe_unused]] const unsigned long long t1 = clk();
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j)
          acc[q >> 1][q & 1][i][j] = load_quads<accv<G>>(ws + ws_index<G>(wave, q, i, j, 0, lane));
#ifdef G9_TIMING
    pin_acc<G>(acc);
    const unsigned long long t2 = clk();
    times.wait += t1 - t0;
    times.load += t2 - t1;
    times.nl += 1;
#endif
  }
  pin_acc<G>(acc);
  mainloop<OP, G>(p, smem, tm, tn, sb, se, acc, false, wb);
  if (se == p.ns) {
    store_tile<OUT, G>(p, smem, tm, tn, acc, epilogue_scale<OP>(p), wb);
    if (sb != 0 && fresh_tid(wb) == 0)
      __hip_atomic_store(p.flags + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    const int tid = fresh_tid(wb), lane = tid & 63, wave = tid >> 6;
    [[maybe_unused]] const unsigned long long t3 = clk();
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j)
          static_for<G::NB>([&](auto B) {
            constexpr int b = decltype(B)::value;
            ws[ws_index<G>(wave, q, i, j, b, lane)] = get_quad<b>(acc[q >> 1][q & 1][i][j]);
          });
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#ifdef G9_TIMING
    __builtin_amdgcn_s_waitcnt(0);
    times.store += clk() - t3;
    times.ns += 1;
#endif
    barrier();
    if (tid == 0)
      __hip_atomic_store(p.flags + tile, (p.epoch << 16) | (u32)se, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <Op OP, int OUT, class G>
G9_DEV void gemm_sk(const GemmParams& p) {
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes<OpInfo<OP>::kScaled>];
  const int G_ = p.sk_ctas;
  // Workgroup ids are dispatched round-robin over the XCDs; give each XCD a
  // contiguous run of ranges so chained neighbours share an L2.
  int cta = blockIdx.x;
  {
    int cm, cn;
    tile_coords(cta, G_, G_, 1, p.num_xcds, 1, cm, cn);
    cta = cm;
  }
  const long long ipt = p.ns;
  const long long total = (long long)p.tiles_m * p.tiles_n * ipt;
  const long long base = total / G_, rem = total % G_;
  const long long u0 = cta * base + min((long long)cta, rem);
  long long u1 = u0 + base + (cta < rem ? 1 : 0);
  SkTimes times;
  sk_stamp(0);
  // Through opaque_s, so the compiler keeps the wave base itself rather than
  // threadIdx.x to re-read it from (a VGPR live through the loop).
  const int wb = (int)opaque_s((u32)__builtin_amdgcn_readfirstlane(threadIdx.x));
  while (u1 > u0) {
    // ipt through opaque_s: the division is redone per segment, not its
    // reciprocal held in a VGPR across the loop.
    const long long ipt_s = (long long)opaque_s((u32)ipt);
    const int tile = __builtin_amdgcn_readfirstlane((int)((u1 - 1) / ipt_s));
    const long long t0 = (long long)tile * ipt;
    const int sb = __builtin_amdgcn_readfirstlane((int)(max(u0, t0) - t0));
    const int se = __builtin_amdgcn_readfirstlane((int)(u1 - t0));
    sk_segment<OP, OUT, G>(p, smem, tile, sb, se, times, wb);
    u1 = t0 + sb;
  }
  sk_stamp(2);
  sk_times_store(times);
}

// ---------------------------------------------------------------------------
// Stream-K with 256x128 tiles (FP16/BF16, 4 waves).
//
// The BASELINE stream-K shapes have fewer 256x256 tiles than CUs (225 and
// 160), where a bit-identical stream-K cannot beat data-parallel: each
// element's K chain is serial, so no range can be shorter than one tile
// chain.  Tiles of 256x128 double the count (450 and 320) so every range
// spans more than a tile.  The tile is two quadrants, A0 x B0 and A1 x B0,
// each computed by the four waves exactly as a 256x256 tile's quadrant (the
// same fragments, snake order and MFMA steps), so every output element sees
// the data-parallel kernel's MFMA sequence and the result is bit-identical to
// it.  Per K stage the tile needs the A0, A1 and B0 sub-buffers (48 KiB):
// three stages are resident (144 KiB), so a stage's DMAs are issued three
// stages ahead.  A stage is two regions of 32 MFMAs per wave:
//   R0: A0 x B0;  reads A1 of this stage and B0 fragments 0-1 of the next;
//       DMAs B0 and half of A0 of the stage three ahead (6 per wave)
//   R1: A1 x B0;  reads A0 of the next stage and B0 fragments 2-3;
//       DMAs the other half of A0 and A1 of the stage three ahead
// Each region waits for its wave's DMAs of three regions earlier (the data it
// reads was issued at least four regions before), then passes the region
// barrier: every wave's reads of the sub-buffers refilled now ended before
// it.  The B registers alternate by stage parity and the slots cycle by 3, so
// the loop body is six stages.  Against the 256x256 tile it issues 1.5x the
// DMAs and LDS reads per MFMA.
// ---------------------------------------------------------------------------
constexpr int kHnTileN = 128;
constexpr int kHnSlots = 3;
// LDS byte offset of sub-buffer X (0: A0, 1: A1, 2: B0) in slot s.
constexpr int hn_off(int X, int s) { return (X * kHnSlots + s) * kSubBytes; }
constexpr int kHnLdsBytes = 3 * kHnSlots * kSubBytes;  // 144 KiB
constexpr int kHnStageRow = kHnTileN * 2 + 16;         // epilogue staging pitch (bytes)
static_assert(kTile * kHnStageRow <= kHnLdsBytes, "staging must fit");
static_assert(hn_off(2, kHnSlots - 1) + kSubBytes <= 65536 * 3, "LDS layout");

template <class G>
using AccH = accv<G>[2][G::FM][G::FN];  // [A half][i][j]

template <Op OP, class G>
struct PipeH {
  static_assert(OP == Op::F16 || OP == Op::BF16, "256x128 stream-K tiles are FP16/BF16");
  static_assert(G::NW == 4 && G::MD == 16, "256x128 stream-K tiles run 4 waves of 16x16 fragments");
  static constexpr int D = G::kDmaPerSub;
  rsrc_t rA[2], rB;
  u32 vA[D], vB[D];
  u32 bA0[G::NC], bA1[G::NC], bB[G::NC];
  u32 lds0, mrow;
  int wave, s_end;
  u32 kshift;

  G9_DEV void init(const GemmParams& p, char* smem, int tm, int tn, int end, int wb) {
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    s_end = __builtin_amdgcn_readfirstlane(end);
    kshift = p.kshift;
    lds0 = (u32)(uintptr_t)to_lds(smem);
    const int tid = fresh_tid(wb);
    const int lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    mrow = lds0 + (u32)wave * (G::kDmaRows * kRowBytes);
    const int wm = wave / G::WN, wn = wave % G::WN;
    const int gi = lane / G::MD, rr = lane % G::MD;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ra = tm * kTile + h * 128;
      const int va = __builtin_amdgcn_readfirstlane(min(max(p.M - ra, 0), 128));
      rA[h] = make_rsrc(p.a + (size_t)ra * p.lda - p.kshift, (u32)va * p.lda + p.kshift);
    }
    const int rb = tn * kHnTileN;
    const int vb = __builtin_amdgcn_readfirstlane(min(max(p.N - rb, 0), 128));
    rB = make_rsrc(p.b + (size_t)rb * p.ldb - p.kshift, (u32)vb * p.ldb + p.kshift);
    // The 256x256 kernel's DMA offsets and row swizzle (Pipe::init).
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int row = G::kDmaRows * wave + 8 * j + (lane >> 3);
      const int ch = (lane & 7) ^ ((row >> 1) & 7);
      vA[j] = (u32)row * p.lda + ch * 16 - 1024u * j;
      vB[j] = (u32)row * p.ldb + ch * 16 - 1024u * j;
    }
    const int sw = (rr >> 1) & 7;
#pragma unroll
    for (int c = 0; c < G::NC; ++c) {
      const int slot = G::chunk(c, gi) ^ sw;
      const u32 ra = (u32)(wm * G::FM * G::MD + rr) * kRowBytes + slot * 16;
      bA0[c] = opaque(lds0 + hn_off(0, 0) + ra);
      bA1[c] = opaque(lds0 + hn_off(1, 0) + ra);
      bB[c] = opaque(lds0 + hn_off(2, 0) + (u32)(wn * G::FN * G::MD + rr) * kRowBytes + slot * 16);
    }
  }
  G9_DEV rsrc_t src(int X) const { return X == 0 ? rA[0] : X == 1 ? rA[1] : rB; }
  G9_DEV u32 stage_off(int stage) const { return stage < s_end ? (u32)stage * kRowBytes : kDeadOff; }
  // 16-byte LDS read number R (fragment R / NC, chunk R % NC) of sub-buffer X.
  template <int X, int SLOT, int R>
  G9_DEV void read_chunk(FragSet<G>& f) const {
    constexpr int NC = G::NC;
    constexpr int imm = SLOT * kSubBytes + (R / NC) * G::MD * kRowBytes;
    static_assert(imm < 65536, "DS offsets are 16 bits");
    const u32 base = X == 0 ? bA0[R % NC] : X == 1 ? bA1[R % NC] : bB[R % NC];
    f[R / NC].c[R % NC] = *(const G9_LDS u32x4*)(uintptr_t)(base + imm);
  }
  template <int X, int SLOT, int J>
  G9_DEV void dma_rows(rsrc_t r, u32 soff, u32 mb) const {
    dma16<J * 1024>(r, (G9_LDS void*)(uintptr_t)(mb + hn_off(X, SLOT)), X < 2 ? vA[J] : vB[J], soff);
  }
  // Every DMA of sub-buffer X for `stage` (the prologue), with the K-tail
  // handling of Pipe::issue.
  template <int X, int SLOT>
  G9_DEV void issue(int stage) const {
    const rsrc_t r = src(X);
    const u32 soff = stage_off(stage);
    if (stage == 0 && kshift != 0) {
      const int lane = fresh_tid_at(wave << 6) & 63;
      static_for<D>([&](auto J) {
        constexpr int j = decltype(J)::value;
        const int row = G::kDmaRows * wave + 8 * j + (lane >> 3);
        const int ch = (lane & 7) ^ ((row >> 1) & 7);
        const u32 v = (u32)ch * 16 < kshift ? kDeadOff : (X < 2 ? vA[j] : vB[j]);
        dma16<j * 1024>(r, (G9_LDS void*)(uintptr_t)(mrow + hn_off(X, SLOT)), v, soff);
      });
      return;
    }
    static_for<D>([&](auto J) { dma_rows<X, SLOT, decltype(J)::value>(r, soff, mrow); });
  }
  template <int X, int SLOT>
  G9_DEV void load(FragSet<G>& f) const {
    constexpr int NF = X < 2 ? G::FM : G::FN;
    static_for<G::NC * NF>([&](auto R) { read_chunk<X, SLOT, decltype(R)::value>(f); });
  }
};

// Region slots of the 256x128 tile: 2 MFMAs before the barrier, the 12 reads
// over the next 15 MFMA slots, the 6 DMAs spread over the region.
struct SlotsH {
  static constexpr int NM = 32, kPre = 2, NQ = NM - kPre, NR = 12, ND = 6;
  static constexpr int read_q(int R) { return R * 15 / NR; }
  static constexpr int dma_q(int J) { return 1 + J * (NQ - 1) / ND; }
};
constexpr int kHnVmWait = 3 * SlotsH::ND;  // DMAs of the three previous regions

// One region: MFMAs of quadrant acc (B fragments bx, A fragments ay); reads of
// A sub-buffer XA / slot SA into na and of B fragments FB0, FB0 + 1 of slot
// SB into nb; DMAs (DPOS 0: B0 and A0 rows 0-15 of the wave's, DPOS 1: A0 rows
// 16-31 and A1) of stage ds into slot SD.
template <Op OP, class G, int XA, int SA, int SB, int FB0, int DPOS, int SD>
G9_DEV void region_h(const PipeH<OP, G>& P, int ds, QAcc<G>& acc, const FragSet<G>& bx, const FragSet<G>& ay,
                     FragSet<G>& na, FragSet<G>& nb) {
  using S = SlotsH;
  static_assert(G::FM * G::NC == 8 && G::NC == 2, "the read table assumes 4 A fragments of 2 chunks");
  __builtin_amdgcn_sched_barrier(0);
  waitcnt<kHnVmWait, 0>();
  const u32 soff = P.stage_off(ds);
  const u32 mb = opaque_s(P.mrow);
  auto slot = [&](auto KC) {
    constexpr int K = decltype(KC)::value;
    constexpr int e = K / (G::FM * G::FN), i = (K / G::FN) % G::FM, j0 = K % G::FN;
    constexpr int j = (i % 2) ? G::FN - 1 - j0 : j0;
    mma<OP, G, e>(acc[i][j], bx[j], ay[i]);
    constexpr int q = K - S::kPre;
    if constexpr (q >= 0) {
      static_for<S::NR>([&](auto RC) {
        constexpr int R = decltype(RC)::value;
        if constexpr (S::read_q(R) == q) {
          if constexpr (R < 8)
            P.template read_chunk<XA, SA, R>(na);
          else
            P.template read_chunk<2, SB, FB0 * G::NC + (R - 8)>(nb);
        }
      });
      static_for<S::ND>([&](auto JC) {
        constexpr int J = decltype(JC)::value;
        if constexpr (S::dma_q(J) == q) {
          constexpr int X = DPOS == 0 ? (J < 4 ? 2 : 0) : (J < 2 ? 0 : 1);
          constexpr int jj = DPOS == 0 ? (J < 4 ? J : J - 4) : (J < 2 ? J + 2 : J - 2);
          P.template dma_rows<X, SD, jj>(P.src(X), soff, mb);
        }
      });
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  static_for<S::kPre>([&](auto K) { slot(K); });
  barrier();
  static_for<S::NM - S::kPre>([&](auto K) { slot(std::integral_constant<int, decltype(K)::value + S::kPre>{}); });
}

template <bool A, class T>
G9_DEV T& pick(T& x, T& y) {
  if constexpr (A)
    return x;
  else
    return y;
}

// Stage K (0..5) of the six-stage body starting at stage s.
template <Op OP, class G, int K>
G9_DEV void stage_h(const PipeH<OP, G>& P, int s, AccH<G>& acc, FragSet<G>& at, FragSet<G>& ab, FragSet<G>& x,
                    FragSet<G>& y) {
  constexpr int sg = K % kHnSlots, sn = (K + 1) % kHnSlots;
  FragSet<G>& bx = pick<K % 2 == 0>(x, y);
  FragSet<G>& nb = pick<K % 2 == 0>(y, x);
  const int ds = s + K + kHnSlots;
  region_h<OP, G, 1, sg, sn, 0, 0, sg>(P, ds, acc[0], bx, at, ab, nb);
  region_h<OP, G, 0, sn, sn, 2, 1, sg>(P, ds, acc[1], bx, ab, at, nb);
}

template <Op OP, class G, int K>
G9_DEV void tail_h(const PipeH<OP, G>& P, int s, int n, AccH<G>& acc, FragSet<G>& at, FragSet<G>& ab,
                   FragSet<G>& x, FragSet<G>& y) {
  if constexpr (K + 1 < 2 * kHnSlots) {
    if (n > K) {
      stage_h<OP, G, K>(P, s, acc, at, ab, x, y);
      tail_h<OP, G, K + 1>(P, s, n, acc, at, ab, x, y);
    }
  }
}

template <class G>
G9_DEV void pin_acc_h(AccH<G>& acc) {
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int j = 0; j < G::FN; ++j) asm volatile("" : "+a"(acc[q][i][j]));
}
template <class G>
G9_DEV void settle_acc_h(AccH<G>& acc) {
  mfma_drain();
  pin_acc_h<G>(acc);
}

// Accumulates stages [s0, s1) of 256x128 tile (tm, tn) into acc; leaves every
// DMA complete and the workgroup synchronised.
template <Op OP, class G>
G9_DEV void mainloop_h(const GemmParams& p, char* smem, int tm, int tn, int s0, int s1, AccH<G>& acc, int wb) {
  constexpr int D = G::kDmaPerSub;
  PipeH<OP, G> P;
  P.init(p, smem, tm, tn, s1, wb);
  // Stages s0 .. s0 + 2 into slots 0 .. 2, each B0, A0, A1 (the order the
  // loop issues them in), then stage s0's B0 and A0 are read.
  P.template issue<2, 0>(s0);
  P.template issue<0, 0>(s0);
  P.template issue<1, 0>(s0);
  P.template issue<2, 1>(s0 + 1);
  P.template issue<0, 1>(s0 + 1);
  P.template issue<1, 1>(s0 + 1);
  P.template issue<2, 2>(s0 + 2);
  P.template issue<0, 2>(s0 + 2);
  P.template issue<1, 2>(s0 + 2);
  waitcnt<7 * D, 0>();
  barrier();
  FragSet<G> at, ab, x, y;
  P.template load<0, 0>(at);
  P.template load<2, 0>(x);
  mfma_drain();
  int s = s0;
  for (; s + 2 * kHnSlots <= s1; s += 2 * kHnSlots)
    static_for<2 * kHnSlots>([&](auto K) { stage_h<OP, G, decltype(K)::value>(P, s, acc, at, ab, x, y); });
  settle_acc_h<G>(acc);
  if (s < s1) {
    tail_h<OP, G, 0>(P, s, s1 - s, acc, at, ab, x, y);
    settle_acc_h<G>(acc);
  }
  waitcnt<0, 0>();
  barrier();
}

// store_tile for a 256x128 tile (staging pitch kHnStageRow).
template <int OUT, class G>
G9_DEV void store_tile_h(const GemmParams& p, char* smem, int tm, int tn, AccH<G>& acc, int wb) {
  const int tid = fresh_tid(wb), lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WN, wn = wave % G::WN;
  const int rr = lane % G::MD, gi = lane / G::MD;
#pragma unroll
  for (int qm = 0; qm < 2; ++qm)
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int j = 0; j < G::FN; ++j) {
        accv<G> f = acc[qm][i][j];
        asm volatile("" : "+v"(f));
        static_for<G::NB>([&](auto B) {
          constexpr int b = decltype(B)::value;
          const int m = qm * 128 + wm * G::FM * G::MD + i * G::MD + rr;
          const int n = wn * G::FN * G::MD + j * G::MD + 4 * G::NG * b + 4 * gi;
          const f32x4 v = get_quad<b>(f);
          const u32x2 h = OUT == OUT_BF16 ? pack4_bf16(v) : pack4_f16(v);
          lds_write8(smem + m * kHnStageRow + n * 2, h);
        });
      }
  waitcnt<0, 0>();
  barrier();
  constexpr int kChunks = kHnTileN / 8;  // 16-byte chunks per row
  constexpr int kRowsPerPass = G::kThreads / kChunks;
  const int ch = tid % kChunks;
  const int col = tn * kHnTileN + ch * 8;
#pragma unroll 4
  for (int pass = 0; pass < kTile / kRowsPerPass; ++pass) {
    const int r = pass * kRowsPerPass + tid / kChunks;
    put_c16(p, tm * kTile + r, col, lds_read16(smem + r * kHnStageRow + ch * 16));
  }
  barrier();
}

// Index (in f32x4) of a wave's fragment in a 256x128 tile's partial.
template <class G>
G9_DEV int ws_index_h(int wave, int q, int i, int j, int lane) {
  return ((wave * (2 * G::FM * G::FN) + (q * G::FM + i) * G::FN + j) * 64 + lane);
}

template <Op OP, int OUT, class G>
G9_DEV void sk_segment_h(const GemmParams& p, char* smem, int tile, int sb, int se, int wb) {
  __builtin_assume(wb >= 0);
  int tm, tn;
  const int tiles_m = (int)opaque_s((u32)p.tiles_m), tiles_n = (int)opaque_s((u32)p.tiles_n);
  tile_coords(tile, tiles_m * tiles_n, tiles_m, tiles_n, 1, (int)opaque_s((u32)p.group_m), tm, tn);
  f32x4* ws = reinterpret_cast<f32x4*>(p.ws) + (size_t)tile * (kTile * kHnTileN / 4);
  AccH<G> acc;
  if (sb == 0) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j) acc[q][i][j] = accv<G>{};
  } else {
    const int tid = fresh_tid(wb), lane = tid & 63, wave = tid >> 6;
    wait_flag(p, tile, (p.epoch << 16) | (u32)sb);
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j) acc[q][i][j] = ws[ws_index_h<G>(wave, q, i, j, lane)];
  }
  pin_acc_h<G>(acc);
  mainloop_h<OP, G>(p, smem, tm, tn, sb, se, acc, wb);
  if (se == p.ns) {
    store_tile_h<OUT, G>(p, smem, tm, tn, acc, wb);
    if (sb != 0 && fresh_tid(wb) == 0)
      __hip_atomic_store(p.flags + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    const int tid = fresh_tid(wb), lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j) ws[ws_index_h<G>(wave, q, i, j, lane)] = acc[q][i][j];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    barrier();
    if (tid == 0)
      __hip_atomic_store(p.flags + tile, (p.epoch << 16) | (u32)se, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The stream-K schedule of gemm_sk over 256x128 tiles (p.tiles_n counts
// 128-column tiles).
template <Op OP, int OUT, class G>
G9_DEV void gemm_sk_h(const GemmParams& p) {
  __shared__ __attribute__((aligned(1024))) char smem[kHnLdsBytes];
  const int G_ = p.sk_ctas;
  int cta = blockIdx.x;
  {
    int cm, cn;
    tile_coords(cta, G_, G_, 1, p.num_xcds, 1, cm, cn);
    cta = cm;
  }
  const long long ipt = p.ns;
  const long long total = (long long)p.tiles_m * p.tiles_n * ipt;
  const long long base = total / G_, rem = total % G_;
  const long long u0 = cta * base + min((long long)cta, rem);
  long long u1 = u0 + base + (cta < rem ? 1 : 0);
  const int wb = (int)opaque_s((u32)__builtin_amdgcn_readfirstlane(threadIdx.x));
  while (u1 > u0) {
    const long long ipt_s = (long long)opaque_s((u32)ipt);
    const int tile = __builtin_amdgcn_readfirstlane((int)((u1 - 1) / ipt_s));
    const long long t0 = (long long)tile * ipt;
    const int sb = __builtin_amdgcn_readfirstlane((int)(max(u0, t0) - t0));
    const int se = __builtin_amdgcn_readfirstlane((int)(u1 - t0));
    sk_segment_h<OP, OUT, G>(p, smem, tile, sb, se, wb);
    u1 = t0 + sb;
  }
}

// ---------------------------------------------------------------------------
// Split-K schedule, for grids with too few tiles to fill the chip.
//
// Each tile's K stages are cut into `split` contiguous segments of near-equal
// length, one workgroup per (segment, tile).  Segment s writes its fp32
// partial tile into the s-th of `split` row-major fp32 matrices of
// tiles_m*256 x tiles_n*256 in the workspace; a second kernel sums the
// segments' partials in segment order, applies the epilogue scale and rounds
// to the output type.  The order of the sum is fixed, so the result is
// deterministic, but it is not bit-identical to the data-parallel kernel,
// whose accumulation runs over K in one chain.
// ---------------------------------------------------------------------------
template <class G>
G9_DEV void store_partial(const GemmParams& p, float* part, int tm, int tn, Acc<G>& acc) {
  const int tid = fresh_tid(), lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WN, wn = wave % G::WN;
  const int rr = lane % G::MD, gi = lane / G::MD;
  const size_t np = (size_t)p.tiles_n * kTile;
#pragma unroll
  for (int qm = 0; qm < 2; ++qm)
#pragma unroll
    for (int qn = 0; qn < 2; ++qn)
#pragma unroll
      for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j)
          static_for<G::NB>([&](auto B) {
            constexpr int b = decltype(B)::value;
            // The quad holds 4 consecutive columns of one row (the layout
            // store_tile also uses), so each store is 16 contiguous bytes.
            const size_t m = (size_t)tm * kTile + qm * 128 + wm * G::FM * G::MD + i * G::MD + rr;
            const size_t n = (size_t)tn * kTile + qn * 128 + wn * G::FN * G::MD + j * G::MD + 4 * G::NG * b + 4 * gi;
            *reinterpret_cast<f32x4*>(part + m * np + n) = get_quad<b>(acc[qm][qn][i][j]);
          });
}

template <Op OP, class G>
G9_DEV void gemm_splitk(const GemmParams& p) {
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes<OpInfo<OP>::kScaled>];
  const int S = p.split;
  // The segments are laid out as S stacked copies of the tile grid, so the
  // XCD remap and GROUP_SIZE_M swizzle keep tiles of one segment (one K range)
  // together on an XCD.
  int vm, tn;
  tile_coords(blockIdx.x, p.tiles_m * S * p.tiles_n, p.tiles_m * S, p.tiles_n, p.num_xcds, p.group_m, vm, tn);
  const int seg = vm / p.tiles_m, tm = vm - seg * p.tiles_m;
  const int sb = (int)((long long)seg * p.ns / S), se = (int)((long long)(seg + 1) * p.ns / S);
  Acc<G> acc;
  zero_acc<G>(acc);
  pin_acc<G>(acc);
  mainloop<OP, G>(p, smem, tm, tn, sb, se, acc);
  float* part = p.ws + (size_t)seg * ((size_t)p.tiles_m * kTile) * ((size_t)p.tiles_n * kTile);
  store_partial<G>(p, part, tm, tn, acc);
}

// One thread per 8 output columns of one row: the segments' partials summed
// in segment order, times the epilogue scale (BF8's per-tensor scales; 1
// otherwise), rounded to 16 bits; rows >= M and columns >= N are not written.
template <int OUT>
G9_DEV void splitk_reduce(const GemmParams& p) {
  const long long np = (long long)p.tiles_n * kTile;
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long m = t / (np / 8);
  const int n = (int)(t - m * (np / 8)) * 8;
  if (m >= p.M || n >= p.N) return;
  const size_t seg = (size_t)p.tiles_m * kTile * (size_t)np;
  const float* src = p.ws + (size_t)m * np + n;
  f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.split; ++s) {
    lo += *reinterpret_cast<const f32x4*>(src + s * seg);
    hi += *reinterpret_cast<const f32x4*>(src + s * seg + 4);
  }
  float scale = 1.f;
  if (p.a_scale) scale *= *p.a_scale;
  if (p.b_scale) scale *= *p.b_scale;
  lo *= scale;
  hi *= scale;
  const u32x2 l = OUT == OUT_BF16 ? pack4_bf16(lo) : pack4_f16(lo);
  const u32x2 h = OUT == OUT_BF16 ? pack4_bf16(hi) : pack4_f16(hi);
  const u32x4 d = {l.x, l.y, h.x, h.y};
  char* dst = p.c + ((size_t)m * p.ldc + n) * 2;
  if (n + 8 <= p.N && ((uintptr_t)dst & 15) == 0) {
    *reinterpret_cast<u32x4*>(dst) = d;
  } else {
    const uint16_t* hv = reinterpret_cast<const uint16_t*>(&d);
    for (int e = 0; e < 8; ++e)
      if (n + e < p.N) reinterpret_cast<uint16_t*>(dst)[e] = hv[e];
  }
}

}  // namespace g9
