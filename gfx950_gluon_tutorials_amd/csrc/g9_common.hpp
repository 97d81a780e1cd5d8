// Shared CDNA4 (gfx950) device helpers for the GEMM kernels.
//
// Everything here is written for gfx950 only: 64-wide waves, buffer
// resources with raw (stride 0) addressing, LDS-DMA (`buffer_load_dwordx4 ...
// lds`), and explicit `s_waitcnt` / `s_barrier` management.  The compiler does
// not track the LDS writes of an LDS-DMA, and `__syncthreads()` drains every
// outstanding global load (vmcnt(0)), so the pipelines below wait on counters by
// hand and synchronise with a bare `s_barrier`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace g9 {

typedef uint32_t u32;
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

#define G9_LDS __attribute__((address_space(3)))
#define G9_DEV __device__ __forceinline__

// Raw buffer resource: base, no stride, `bytes` valid bytes.  Accesses at an
// offset >= bytes return zero (loads) or are dropped (stores).  Word 3 is the
// gfx9-family default descriptor format.
G9_DEV rsrc_t make_rsrc(const void* base, u32 bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Cache-policy bits of the operand DMAs (gfx950 CPol: bit 0 sc0, bit 1 nt,
// bit 4 sc1); a build option.
#ifndef G9_DMA_CPOL
#define G9_DMA_CPOL 0
#endif

// One LDS-DMA of 16 bytes per lane: lane i writes lds + IMM + 16*i (the whole
// wave writes one contiguous KiB), reading global base + voff + soff + IMM.
// The instruction's immediate offset moves the global and the LDS address
// alike, so DMAs IMM bytes apart in both can share one M0 (the LDS base).
template <int IMM = 0>
G9_DEV void dma16(rsrc_t r, G9_LDS void* lds, u32 voff, u32 soff) {
  static_assert(IMM >= 0 && IMM < 4096, "MUBUF immediate offsets are 12 bits");
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, (int)voff, (int)soff, IMM, G9_DMA_CPOL);
}
// Same with 4 bytes per lane (a wave writes 256 contiguous bytes).
G9_DEV void dma4(rsrc_t r, G9_LDS void* lds, u32 voff, u32 soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 4, (int)voff, (int)soff, 0, G9_DMA_CPOL);
}

// s_waitcnt with vmcnt(VM) and lgkmcnt(LG); expcnt is left unconstrained.
// gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4]<<14.
template <int VM, int LG>
G9_DEV void waitcnt() {
  static_assert(VM >= 0 && VM < 64 && LG >= 0 && LG < 16, "counter out of range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (LG << 8) | ((VM >> 4) << 14));
}

// Workgroup barrier without the memory fence `__syncthreads()` implies.  The
// scheduling fences keep the compiler from moving LDS traffic across it.
G9_DEV void barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

G9_DEV u32x4 lds_read16(const char* p) { return *reinterpret_cast<const u32x4*>(p); }
G9_DEV u32x2 lds_read8(const char* p) { return *reinterpret_cast<const u32x2*>(p); }
G9_DEV void lds_write8(char* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }
G9_DEV G9_LDS void* to_lds(char* p) { return (G9_LDS void*)(p); }

// Instruction-class masks for __builtin_amdgcn_sched_group_barrier.
enum : int {
  SG_VALU = 0x2,
  SG_SALU = 0x4,
  SG_MFMA = 0x8,
  SG_VMEM = 0x10,
  SG_VMEM_RD = 0x20,
  SG_DS_RD = 0x100,
  SG_DS_WR = 0x200,
  SG_TRANS = 0x400,  // transcendental (v_exp, v_log, ...): not in SG_VALU
};

// XCD-aware tile remap followed by a GROUP_SIZE_M swizzle.  Workgroups are
// dispatched round-robin over the 8 XCDs; the remap gives each XCD one
// contiguous run of tile ids, and the swizzle walks each run GROUP_M tile rows
// at a time (column-major inside a group) so tiles sharing A rows or B columns
// sit on the same L2.
// Follows kernels/gemm/utils/common.py:38-83 (get_pids).
G9_DEV void tile_coords(int pid, int grid_mn, int tiles_m, int tiles_n, int num_xcds, int group_m,
                        int& pid_m, int& pid_n) {
  if (num_xcds != 1) {
    const int per_xcd = (grid_mn + num_xcds - 1) / num_xcds;
    int tall = grid_mn % num_xcds;
    tall = tall == 0 ? num_xcds : tall;
    const int xcd = pid % num_xcds;
    const int local = pid / num_xcds;
    pid = xcd < tall ? xcd * per_xcd + local
                     : tall * per_xcd + (xcd - tall) * (per_xcd - 1) + local;
  }
  if (group_m == 1) {
    pid_m = pid / tiles_n;
    pid_n = pid % tiles_n;
  } else {
    const int in_group = group_m * tiles_n;
    const int gid = pid / in_group;
    const int first_m = gid * group_m;
    const int gsize = min(tiles_m - first_m, group_m);
    const int r = pid % in_group;
    pid_m = first_m + r % gsize;
    pid_n = r / gsize;
  }
}

// Round-to-nearest-even conversions of four fp32 values packed as 4 x 16 bit.
G9_DEV u32x2 pack4_f16(f32x4 v) {
  f16x4 h = __builtin_convertvector(v, f16x4);
  return __builtin_bit_cast(u32x2, h);
}
G9_DEV u32x2 pack4_bf16(f32x4 v) {
  bf16x4 h = __builtin_convertvector(v, bf16x4);
  return __builtin_bit_cast(u32x2, h);
}

}  // namespace g9
