// LDS tiles for MFMA operands on gfx950: 64-row bf16 tiles filled by direct-to-LDS loads,
// kswz-swizzled row-major, and the LDS transpose loads (ds_read_b64_tr_b16) that read their
// columns as MFMA operands. Shared by the attention and the skinny TN GEMM kernels.
#pragma once
#include "common.h"

// Row-major [64 keys x D] tiles filled by direct global->LDS loads (16 bytes per lane). The
// 16-byte chunk c of row r sits at slot c ^ kswz(r). For D = 128 (256-byte rows, one full pass
// over the 64 banks) kswz rotates the row's low four bits: it is a bijection on any 16
// consecutive rows (16-byte fragment reads: 16 rows, one chunk, per LDS cycle) and its two high
// bits differ across any 4 aligned rows (transpose loads: 4 rows x 4 consecutive chunks per half
// wave), so both read patterns hit distinct banks. kswz(r + 16) = kswz(r). D = 32 tiles
// (64-byte rows) need no swizzle: the half wave of a transpose load reads 4 consecutive whole
// rows, 256 contiguous bytes.
template <int D> __device__ __forceinline__ int kswz(int r) {
  return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : D == 32 ? 0 : ((r >> 1) & 7);
}

// A operand of a 16-key MFMA step read straight from a row-major, kswz-swizzled [64 keys x D]
// tile with two LDS transpose loads (ds_read_b64_tr_b16). Within each 16-lane group the load
// hands result lane j the (j % 4)-th element of the 8-byte rows supplied by source lanes j / 4 +
// {0, 4, 8, 12}. Source lane s of group G supplies row r0 = 16p + 4 * (G >> 1) + s / 4 (then
// r0 + 8), columns c = 32 tt + 16 * (G & 1) + 4 * (s % 4) .. + 3, so result lane (lq, g) receives
// dim 32 tt + lq of keys 16p + 4g + {0..3} and 16p + 8 + 4g + {0..3}: the accumulator's key order.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Element offsets (within a [64 keys x D] tile) of the two rows lane `lane` supplies for operand
// (tt, p = 0); operand p adds 16 * p * D (the kswz swizzle does not depend on p).
template <int D>
__device__ __forceinline__ int2 tr_frag_off(int tt, int lane) {
  const int G = lane >> 4, sl = lane & 15;
  const int c = tt * 32 + 16 * (G & 1) + 4 * (sl & 3);
  const int r0 = 4 * (G >> 1) + (sl >> 2);
  return make_int2(r0 * D + (((c >> 3) ^ kswz<D>(r0)) << 3) + (c & 7),
                   (r0 + 8) * D + (((c >> 3) ^ kswz<D>(r0 + 8)) << 3) + (c & 7));
}

// Transpose loads of operand p from LDS byte addresses a (rows at p = 0): the step's 16-row
// displacement is the instruction's immediate offset. They are written as inline assembly: the
// compiler would otherwise wait for every direct-to-LDS load still in flight (the next tile's)
// before the first of them, since it cannot tell the stages apart. The caller waits for them
// (s_waitcnt lgkmcnt with the results as operands) before using the results.
template <int OFF>
__device__ __forceinline__ void tr_issue_at(uint2 a, u32x2_t& lo, u32x2_t& hi) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(lo) : "v"(a.x), "i"(OFF));
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(hi) : "v"(a.y), "i"(OFF));
}
// BASE: a further constant byte displacement (e.g. the LDS stage), folded into the immediate.
template <int D, int BASE = 0>
__device__ __forceinline__ void tr_issue_p(uint2 a, int p, u32x2_t& lo, u32x2_t& hi) {
  constexpr int STEP = 16 * D * 2;   // bytes per 16 key rows
  static_assert(BASE + 3 * STEP < 65536, "LDS immediate offset range");
  if (p == 0) tr_issue_at<BASE>(a, lo, hi);
  else if (p == 1) tr_issue_at<BASE + STEP>(a, lo, hi);
  else if (p == 2) tr_issue_at<BASE + 2 * STEP>(a, lo, hi);
  else tr_issue_at<BASE + 3 * STEP>(a, lo, hi);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ bf16x8_t tr_join(u32x2_t lo, u32x2_t hi) {
  return __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// Waits for every LDS load in flight; the transpose-load results of two 16-key steps pass
// through the wait as operands, so nothing reads them before it.
template <int NDT>
__device__ __forceinline__ void tr_wait_all(u32x2_t (&lo)[2][NDT], u32x2_t (&hi)[2][NDT]) {
  if constexpr (NDT == 4)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(lo[0][0]), "+v"(hi[0][0]), "+v"(lo[0][1]), "+v"(hi[0][1]), "+v"(lo[0][2]), "+v"(hi[0][2]),
                   "+v"(lo[0][3]), "+v"(hi[0][3]), "+v"(lo[1][0]), "+v"(hi[1][0]), "+v"(lo[1][1]), "+v"(hi[1][1]),
                   "+v"(lo[1][2]), "+v"(hi[1][2]), "+v"(lo[1][3]), "+v"(hi[1][3]));
  else
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(lo[0][0]), "+v"(hi[0][0]), "+v"(lo[0][1]), "+v"(hi[0][1]), "+v"(lo[1][0]), "+v"(hi[1][0]),
                   "+v"(lo[1][1]), "+v"(hi[1][1]));
}

// As tr_wait_all, for the transpose-load results of one 16-key step.
template <int NDT>
__device__ __forceinline__ void tr_wait_one(u32x2_t (&lo)[NDT], u32x2_t (&hi)[NDT]) {
  if constexpr (NDT == 4)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(lo[0]), "+v"(hi[0]), "+v"(lo[1]), "+v"(hi[1]), "+v"(lo[2]), "+v"(hi[2]), "+v"(lo[3]), "+v"(hi[3]));
  else
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo[0]), "+v"(hi[0]), "+v"(lo[1]), "+v"(hi[1]));
}

// Byte offset, within a 64-row tile of a row-major [rows, ld] bf16 matrix (columns [col0,
// col0 + D)), of the 16 bytes this lane moves in its first direct-to-LDS load of the tile. Load i
// adds i * NW * RPI rows: kswz repeats every 16 rows, so the swizzled chunk is the same for all i.
template <int D, int NW = 4>
__device__ __forceinline__ uint32_t dma_lane_off(int64_t ld, int col0, int wid, int lane) {
  constexpr int CPR = D / 8, RPI = 64 / CPR;
  static_assert((NW * RPI) % 16 == 0, "the swizzle must repeat across a lane's loads");
  const int rl = lane / CPR, slot = lane % CPR;
  const int r = wid * RPI + rl;
  return (uint32_t)(((int64_t)r * ld + col0 + ((slot ^ kswz<D>(r)) << 3)) * 2);
}

// One 64-row tile of a row-major [rows, ld] bf16 matrix via buffer loads straight into LDS, at
// the per-lane offsets of dma_lane_off. The buffer resource starts at row k0 and covers rows
// [k0, kend), so rows past kend read as zeros without any clamping arithmetic (their keys are
// masked).
template <int D, int NW = 4>
__device__ __forceinline__ void dma_tile(const bf16_t* src, int64_t ld, uint32_t lane_off, int k0, int kend,
                                         bf16_t* dst, int wid) {
  constexpr int CPR = D / 8, RPI = 64 / CPR, INS = 64 / (RPI * NW);
  static_assert(INS >= 1, "tile too small for the wave count");
  // The tile's source, start row and row count are workgroup-uniform; reading them through
  // readfirstlane keeps the buffer resource in SGPRs (a resource the compiler cannot prove
  // uniform is issued through a per-load waterfall loop).
  const int nrows = __builtin_amdgcn_readfirstlane(max(0, min(kend - k0, 64)));
  const uintptr_t base = (uintptr_t)(src + (int64_t)k0 * ld);
  const uintptr_t ubase = ((uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32)) << 32) |
                          (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  const int64_t uld = ((int64_t)__builtin_amdgcn_readfirstlane((int)(ld >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)ld);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)ubase, (short)0, (int)((int64_t)nrows * uld * 2), 0x00020000);
  const uint32_t step = (uint32_t)uld * (2 * NW * RPI);
#pragma unroll
  for (int i = 0; i < INS; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + (i * NW + wid) * RPI * D),
                                             16, lane_off + i * step, 0, 0, 0);
}

