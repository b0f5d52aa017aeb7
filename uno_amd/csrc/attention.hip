// Block-diffusion attention, forward and backward (bf16 MFMA and fp32 kernels).
//
// Visibility is given per query row as key intervals over two K/V sources:
//   source 1 = clean-stream K/V, keys [lo1, hi1);  source 2 = noisy-stream K/V, keys [lo2, hi2)
// which expresses every pattern of the step exactly (bd mask contract, A.4 of the survey):
//   clean query i (segment start s):  src1 [s, i+1)                      -- causal clean stream
//   noisy query i in block k:         src1 [s, s+k*b)  +  src2 [s+k*b, s+min((k+1)b, len))
// Row tables are int32[8] per row: lo1, hi1, lo2, hi2, qlo2, qhi2, 0, 0, where [qlo2, qhi2) is
// the range of source-2 query rows that may see this row as a key (used by dK/dV).
//
// The bf16 kernels compute S^T = K Q^T with v_mfma_f32_32x32x16_bf16 so that each lane owns
// one query (its softmax statistics are per-lane scalars); P^T is fed to the P.V product
// directly from the accumulator registers, with the MFMA k-index permuted to match the
// accumulator's key order. K tiles are staged row-major in LDS and V tiles transposed.
// Tiles outside a wave's key range are skipped; tiles wholly inside every query's interval
// run without evaluating the mask. Softmax runs in the exp2 domain; LSE is stored as
// log2-sum-exp2 of the scaled scores (lse2) for the backward pass.
#include "common.h"
#include "lds_tile.h"

#include <stdlib.h>
#include <type_traits>

struct AttnArgs {
  const void* Q; int64_t ldq;          // [Mq, Hq*D]
  const void* K1; int64_t ldk1;        // source 1 keys  [Mk1, Hkv*D]
  const void* V1; int64_t ldv1;
  const void* K2; int64_t ldk2;        // source 2 keys (may be null)
  const void* V2; int64_t ldv2;
  const int32_t* iv;                   // [Mq, 8] query intervals
  void* O; int64_t ldo;                // [Mq, Hq*D]
  float* LSE;                          // [Mq, Hq]
  // backward
  const void* dO; int64_t lddo;
  float* Dsum;                         // [Mq, Hq] rowsum(dO * O), written by the dQ kernel
  void* dQ; int64_t lddq;
  const int32_t* ivk;                  // [Mk2, 8] key-side table (qlo2, qhi2 at 4, 5)
  void* dK; int64_t lddk;              // [Mk2, Hkv*D]
  void* dV; int64_t lddv;
  int Mq, Mk2, Hq, Hkv;
  int q_mod;                           // > 0: query row i reads Q row i % q_mod (split-key decode)
  int grad_f32;                        // bf16 kernels: dQ and dK stored as fp32 (dV keeps bf16)
  // bf16 kernels with qkn_out set: instead of dQ / dK, the gradient of the q/k projection before
  // the q/k RMSNorm and RoPE (their backward applied to the fp32 dQ / dK accumulators), written into
  // the q / k column blocks of qkn_out [Mq, (Hq + 2 Hkv) D]; the q/k head columns of qkn_pre
  // [Mq, (Hq + Hkv) D] are the pre-norm values (bf16), qkn_rstd [Mq, Hq + Hkv] their 1/rms, and
  // qkn_cos / qkn_sin [qkn_P, D/2] the angles at each row's position qkn_pos. No norm when qkn_wq is
  // null (RoPE only).
  bf16_t* qkn_out; int64_t ld_qkn_out;
  const bf16_t* qkn_pre; int64_t ld_qkn_pre;
  const float* qkn_rstd;
  const bf16_t* qkn_wq; const bf16_t* qkn_wk;
  const int64_t* qkn_pos;
  const float* qkn_cos; const float* qkn_sin;
  int qkn_P;
  float scale;                         // d^-0.5
  float scale_log2;                    // d^-0.5 * log2(e)
};

__device__ __forceinline__ bf16x8_t ld_bf16x8(const bf16_t* p) { return *(const bf16x8_t*)p; }

// Backward of y = RoPE(w * x * rstd) (q/k RMSNorm then rotate_half RoPE, modeling_qwen3.py:140-160,
// 237-253) for one row and head, on the fp32 gradient dy held as the MFMA accumulators of the
// dQ / dK kernels: lane (g, row) holds dims c = 32 t + 8 j4 + 4 g + e of acc[t][4 j4 + e] (times
// scale), so a dim's RoPE partner c +- D/2 is block t ^ (NDT/2) of the same lane and the other half
// of the row sits in lane ^ 32. Writes r (g - xhat mean(g xhat)) with g = w * RoPE^-1(dy) (or
// RoPE^-1(dy) without the norm) as bf16 at dst[c]; pre / rs: the row's pre-norm head and 1/rms;
// cs / sn: the row's angle-table rows. Lanes with valid false take part in the shuffle only.
template <int D>
__device__ __forceinline__ void qknorm_rope_bwd_acc(const f32x16_t (&acc)[D / 32], float scale, int g, bool valid,
                                                    const bf16_t* pre, float rs, const bf16_t* wn, const float* cs,
                                                    const float* sn, bf16_t* dst) {
  constexpr int NDT = D / 32, HT = NDT / 2;
  // every input load first (independent of each other), then the arithmetic
  float4 cv[HT][4], sv[HT][4];
  uint2 xw[NDT][4], ww[NDT][4];
#pragma unroll
  for (int t = 0; t < HT; ++t)
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4) {
      const int f = 32 * t + 8 * j4 + 4 * g;                 // angle index of the lower dim (= c mod D/2)
      cv[t][j4] = valid ? *(const float4*)(cs + f) : make_float4(0.f, 0.f, 0.f, 0.f);
      sv[t][j4] = valid ? *(const float4*)(sn + f) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  if (wn != nullptr) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const int c = 32 * t + 8 * j4 + 4 * g;
        xw[t][j4] = valid ? *(const uint2*)(pre + c) : make_uint2(0, 0);
        ww[t][j4] = valid ? *(const uint2*)(wn + c) : make_uint2(0, 0);
      }
  }
  float gv[NDT][16];
#pragma unroll
  for (int t = 0; t < HT; ++t)
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4) {
      const float c4[4] = {cv[t][j4].x, cv[t][j4].y, cv[t][j4].z, cv[t][j4].w};
      const float s4[4] = {sv[t][j4].x, sv[t][j4].y, sv[t][j4].z, sv[t][j4].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = acc[t][4 * j4 + e] * scale, hi = acc[t + HT][4 * j4 + e] * scale;
        // inverse rotation: dn_c = dy_c cos + dy_{c+h} sin (lower), dy_c cos - dy_{c-h} sin (upper)
        gv[t][4 * j4 + e] = lo * c4[e] + hi * s4[e];
        gv[t + HT][4 * j4 + e] = hi * c4[e] - lo * s4[e];
      }
    }
  if (wn != nullptr) {
    float xh[NDT][16];
    float dot = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const uint2 xv = xw[t][j4], wv = ww[t][j4];
        const float x4[4] = {__uint_as_float(xv.x << 16), __uint_as_float(xv.x & 0xffff0000u),
                             __uint_as_float(xv.y << 16), __uint_as_float(xv.y & 0xffff0000u)};
        const float w4[4] = {__uint_as_float(wv.x << 16), __uint_as_float(wv.x & 0xffff0000u),
                             __uint_as_float(wv.y << 16), __uint_as_float(wv.y & 0xffff0000u)};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xh[t][4 * j4 + e] = x4[e] * rs;
          gv[t][4 * j4 + e] *= w4[e];
          dot += gv[t][4 * j4 + e] * xh[t][4 * j4 + e];
        }
      }
    dot += __shfl_xor(dot, 32, 64);
    dot /= (float)D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) gv[t][r] = rs * (gv[t][r] - xh[t][r] * dot);
  }
  if (!valid) return;
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4)
      *(uint2*)(dst + 32 * t + 8 * j4 + 4 * g) =
          make_uint2(pack2_bf16(gv[t][4 * j4], gv[t][4 * j4 + 1]), pack2_bf16(gv[t][4 * j4 + 2], gv[t][4 * j4 + 3]));
}

__device__ __forceinline__ bf16x8_t pack_bf16x8(const float* v) {
  uint4 u = make_uint4(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]), pack2_bf16(v[4], v[5]), pack2_bf16(v[6], v[7]));
  return __builtin_bit_cast(bf16x8_t, u);
}

// 2^x with the bare hardware instruction (inputs here are <= 8; results that would be
// denormal flush towards zero, which is immaterial for softmax weights).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

// Interval bounds reduced over a workgroup's 4 waves. Empty intervals are ignored.
struct Bounds { int lo, hi, maxlo, minhi; };

__device__ __forceinline__ Bounds wave_bounds(bool valid, int lo, int hi) {
  const bool use = valid && lo < hi;
  // Wave-wide reductions, so uniform: readfirstlane lets the tile tests branch on scalars.
  Bounds b;
  b.lo = __builtin_amdgcn_readfirstlane(wave_min_i(use ? lo : INT_MAX));
  b.hi = __builtin_amdgcn_readfirstlane(wave_max_i(use ? hi : INT_MIN));
  // for the "whole tile visible" test every valid query counts (an empty one forces the mask)
  b.maxlo = __builtin_amdgcn_readfirstlane(wave_max_i(valid ? lo : INT_MIN));
  b.minhi = __builtin_amdgcn_readfirstlane(wave_min_i(valid ? (lo < hi ? hi : INT_MIN) : INT_MAX));
  return b;
}

// Workgroup-wide (lo, hi) of the 4 waves' bounds, returned by value (x = lo, y = hi).
__device__ __forceinline__ int2 wg_bounds(const Bounds& w, int* sh) {
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sh[wid * 2] = w.lo; sh[wid * 2 + 1] = w.hi; }
  __syncthreads();
  const int lo = min(min(sh[0], sh[2]), min(sh[4], sh[6]));
  const int hi = max(max(sh[1], sh[3]), max(sh[5], sh[7]));
  __syncthreads();
  return make_int2(__builtin_amdgcn_readfirstlane(lo), __builtin_amdgcn_readfirstlane(hi));
}

constexpr int ATT_BK = 64;     // keys per tile

// max(v[l], v[l ^ 32]) in every lane l, by swapping the two 32-lane halves in registers
// (v_permlane32_swap) instead of a round trip through the LDS crossbar.
__device__ __forceinline__ float half_swap_max(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// MFMA fragment (row r, 16-byte chunk c) of a swizzled row-major tile.
template <int D>
__device__ __forceinline__ bf16x8_t ld_frag(const bf16_t* tile, int r, int c) {
  return *(const bf16x8_t*)&tile[r * D + ((c ^ kswz<D>(r)) << 3)];
}


__device__ __forceinline__ Bounds merge_bounds(const Bounds& a, const Bounds& b) {
  Bounds r;
  r.lo = min(a.lo, b.lo); r.hi = max(a.hi, b.hi);
  r.maxlo = max(a.maxlo, b.maxlo); r.minhi = min(a.minhi, b.minhi);
  return r;
}

// ---------------------------------------------------------------------------------------
// Forward, bf16: one workgroup = 256 queries of one q-head; each wave owns 64 queries as two
// groups of 32 (one per MFMA column block), so every K/V fragment read from LDS feeds two MFMAs.
// ---------------------------------------------------------------------------------------
template <int D, int QG>
__global__ __launch_bounds__(256, QG == 1 ? 2 : 1) void attn_fwd_bf16_kernel(const AttnArgs p) {
  constexpr int BK = ATT_BK, NKS = D / 16, NDT = D / 32, BQ = 128 * QG;
  // Dynamic LDS: K and V tiles [2][64*D] each, double-buffered, filled by direct-to-LDS loads;
  // the P.V operand is read from the row-major V tile with LDS transpose loads.
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];
  bf16_t* Ks = smem;
  bf16_t* Vs = smem + 2 * BK * D;
  __shared__ int sh[8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, lq = lane & 31;
  const int nqt = (p.Mq + BQ - 1) / BQ;
  const int lin = xcd_remap(blockIdx.x, nqt * p.Hq);
  // K/V-head-major order: each XCD takes a contiguous range of K/V heads, and the query heads
  // sharing a K/V head are interleaved q tile by q tile, so the workgroups running together on an
  // XCD stream the same K/V tiles from its L2 at the same time (clean 4 x 4096 forward: 0.84 ms
  // with the q-tile-major order, 0.71 head-major, 0.65 this way). The q tiles run from the last
  // to the first: with causal-like masks the late tiles carry the most key tiles, so the heaviest
  // workgroups start first and the tail is light.
  const int rep = p.Hq / p.Hkv, kvh = lin / (nqt * rep), rem = lin % (nqt * rep);
  const int h = kvh * rep + rem % rep, qt = nqt - 1 - rem / rep;
  int qrow[QG];
  bool qvalid[QG];
  int4 ivq[QG];
  const bf16_t* Q = (const bf16_t*)p.Q;
  bf16x8_t qreg[QG][NKS];
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    qrow[qg] = qt * BQ + w * (32 * QG) + qg * 32 + lq;
    qvalid[qg] = qrow[qg] < p.Mq;
    ivq[qg] = qvalid[qg] ? *(const int4*)(p.iv + (int64_t)qrow[qg] * 8) : make_int4(0, 0, 0, 0);
    const int qsrc = p.q_mod > 0 ? qrow[qg] % p.q_mod : qrow[qg];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qreg[qg][ks] = qvalid[qg] ? ld_bf16x8(Q + (int64_t)qsrc * p.ldq + h * D + ks * 16 + g * 8)
                                : __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
  }

  float m_run[QG], l_run[QG];
  f32x16_t oacc[QG][NDT];
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    m_run[qg] = -INFINITY;
    l_run[qg] = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[qg][t][r] = 0.f;
  }

  // Tile walk over both sources: tiles [0, n1) come from source 1, [n1, n1 + n2) from source 2.
  const bool has2 = p.K2 != nullptr;
  Bounds wb1 = wave_bounds(qvalid[0], ivq[0].x, ivq[0].y);
  Bounds wb2 = wave_bounds(has2 && qvalid[0], ivq[0].z, ivq[0].w);
#pragma unroll
  for (int qg = 1; qg < QG; ++qg) {
    wb1 = merge_bounds(wb1, wave_bounds(qvalid[qg], ivq[qg].x, ivq[qg].y));
    wb2 = merge_bounds(wb2, wave_bounds(has2 && qvalid[qg], ivq[qg].z, ivq[qg].w));
  }
  const int2 r1 = wg_bounds(wb1, sh), r2 = wg_bounds(wb2, sh);
  const int kb1 = r1.x, ke1 = r1.y, kb2 = r2.x, ke2 = r2.y;
  const int n1 = kb1 < ke1 ? (ke1 - (kb1 / BK) * BK + BK - 1) / BK : 0;
  const int n2 = (has2 && kb2 < ke2) ? (ke2 - (kb2 / BK) * BK + BK - 1) / BK : 0;
  const int nt = n1 + n2;
  const bf16_t* K1 = (const bf16_t*)p.K1;
  const bf16_t* V1 = (const bf16_t*)p.V1;
  const bf16_t* K2 = (const bf16_t*)p.K2;
  const bf16_t* V2 = (const bf16_t*)p.V2;
  const int wid = __builtin_amdgcn_readfirstlane(w);
  // Tile t streams into K and V stage t & 1; every thread issues its loads of tile t+1 right
  // after the barrier that ends tile t-1 (whose stage they overwrite), so they fly during tile
  // t's math.
  // The source is chosen arithmetically (f2 in {0, 1}), not with selects between variables:
  // the compiler would otherwise turn those into selected addresses of stack/kernarg memory.
  const uintptr_t k1a = (uintptr_t)K1, v1a = (uintptr_t)V1;
  const uintptr_t kd = (uintptr_t)K2 - k1a, vd = (uintptr_t)V2 - v1a;
  const int64_t ldkd = p.ldk2 - p.ldk1, ldvd = p.ldv2 - p.ldv1;
  const int kt1 = (kb1 / BK) * BK, kt2 = (kb2 / BK) * BK - n1 * BK;
  // Per-lane byte offsets of the direct-to-LDS loads, one per source tensor, fixed for the walk.
  const uint32_t ko1 = dma_lane_off<D>(p.ldk1, kvh * D, wid, lane), vo1 = dma_lane_off<D>(p.ldv1, kvh * D, wid, lane);
  const uint32_t ko2 = has2 ? dma_lane_off<D>(p.ldk2, kvh * D, wid, lane) : 0u;
  const uint32_t vo2 = has2 ? dma_lane_off<D>(p.ldv2, kvh * D, wid, lane) : 0u;
  auto fetch = [&](int t, int stage) {
    const int f2 = t >= n1 ? 1 : 0;
    const int fkt = (f2 ? kt2 : kt1) + t * BK;
    const int fke = ke1 + f2 * (ke2 - ke1);
    dma_tile<D>((const bf16_t*)(k1a + f2 * kd), p.ldk1 + f2 * ldkd, f2 ? ko2 : ko1, fkt, fke, Ks + stage * BK * D, wid);
    dma_tile<D>((const bf16_t*)(v1a + f2 * vd), p.ldv1 + f2 * ldvd, f2 ? vo2 : vo1, fkt, fke, Vs + stage * BK * D, wid);
  };
  // Per-lane LDS offsets, fixed for the whole walk: K fragments (row lq, chunk 2 ks + g) and the
  // rows this lane supplies to the V transpose loads.
  int koff[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) koff[ks] = lq * D + (((ks * 2 + g) ^ kswz<D>(lq)) << 3);
  // LDS byte addresses of the V transpose loads in stage 0; the stage and the 16-key step are
  // immediate offsets (the tile loop below is unrolled over the two stages).
  uint2 vaddr[NDT];
  const uint32_t vbase0 = lds_addr(Vs);
#pragma unroll
  for (int tt = 0; tt < NDT; ++tt) {
    const int2 o = tr_frag_off<D>(tt, lane);
    vaddr[tt] = make_uint2(vbase0 + 2 * o.x, vbase0 + 2 * o.y);
  }
  if (nt > 0) fetch(0, 0);
  // One K/V tile in LDS stage ST (t & 1), so every stage offset is a compile-time constant.
  auto tile = [&](const int t, auto stc) {
    constexpr int ST = decltype(stc)::value;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();                       // K(t), V(t) in LDS; every wave is done with tile t-1
    if (t + 1 < nt) fetch(t + 1, ST ^ 1);
    const bf16_t* Kc = Ks + ST * BK * D;
    const bool s2 = t >= n1;
    const int kt = s2 ? (kb2 / BK) * BK + (t - n1) * BK : (kb1 / BK) * BK + t * BK;
    const int w_lo = s2 ? wb2.lo : wb1.lo, w_hi = s2 ? wb2.hi : wb1.hi;
    const int w_maxlo = s2 ? wb2.maxlo : wb1.maxlo, w_minhi = s2 ? wb2.minhi : wb1.minhi;
    if (kt >= w_hi || kt + BK <= w_lo) return;
    const bool full = kt >= w_maxlo && kt + BK <= w_minhi;
    // Scores of both 32-key halves (kk). All K fragments of the tile are read before the first
    // product, so the two MFMA chains run back to back instead of each MFMA waiting for its read.
    f32x16_t sacc[2][QG];
    {
      bf16x8_t kf[2][NKS];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) kf[kk][ks] = *(const bf16x8_t*)(Kc + kk * 32 * D + koff[ks]);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int qg = 0; qg < QG; ++qg) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[kk][qg][r] = 0.f;
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks)
            sacc[kk][qg] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kk][ks], qreg[qg][ks], sacc[kk][qg], 0, 0, 0);
        }
#pragma unroll
      for (int i = 0; i < 2 * NKS; ++i) __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
#pragma unroll
      for (int i = 0; i < 2 * NKS * QG; ++i) __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!full) {   // wave-uniform: only tiles that cut through some query's interval
#pragma unroll
      for (int qg = 0; qg < QG; ++qg) {
        const int lo = s2 ? ivq[qg].z : ivq[qg].x, hi = s2 ? ivq[qg].w : ivq[qg].y;
        // key in [lo, hi)  <=>  (unsigned)(key - lo) < (unsigned)(hi - lo)
        const uint32_t span = (uint32_t)max(hi - lo, 0);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int d0 = kt + kk * 32 + 4 * g - lo;
#pragma unroll
          for (int j = 0; j < 16; ++j)
            sacc[kk][qg][j] = (uint32_t)(d0 + 8 * (j >> 2) + (j & 3)) < span ? sacc[kk][qg][j] : -INFINITY;
        }
      }
    }
    // V operands of the two 16-key steps of half kk ([kk][step][tt]).
    u32x2_t vlo[2][2][NDT], vhi[2][2][NDT];
    auto issue_v = [&](int kk) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int tt = 0; tt < NDT; ++tt)
          tr_issue_p<D, ST * BK * D * 2>(vaddr[tt], kk * 2 + hh, vlo[kk][hh][tt], vhi[kk][hh][tt]);
    };
    issue_v(0);   // in flight during the softmax
    // One running-max update per tile. Raw scores; the scale (> 0) is applied inside the
    // exponent: p = 2^(s*scale_log2 - m).
    float neg_m[QG];
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) {
      float tmax = sacc[0][qg][0];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = kk ? 0 : 1; j < 16; ++j) tmax = fmaxf(tmax, sacc[kk][qg][j]);
      tmax = half_swap_max(tmax) * p.scale_log2;
      // Lazy rescaling: the running max moves only when a row's max exceeds it by more than
      // 8 (log2 units), so weights stay <= 2^8 and most tiles skip rescaling the accumulators.
      const bool grow = tmax > m_run[qg] + 8.f;
      if (__any(grow)) {
        const float m_new = grow ? fmaxf(m_run[qg], tmax) : m_run[qg];
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run[qg] - m_new);
        l_run[qg] *= alpha;
#pragma unroll
        for (int tt = 0; tt < NDT; ++tt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[qg][tt][r] *= alpha;
        m_run[qg] = m_new;
      }
      // Branch-free when nothing is visible yet (m_run = -inf): every lane keeps feeding the
      // shared MFMAs, with weights 2^-inf = 0.
      neg_m[qg] = m_run[qg] == -INFINITY ? 0.f : -m_run[qg];
    }
    // Weights of half kk, packed to bf16 as the B operands of its two 16-key steps.
    bf16x8_t pb[2][2][QG];
    auto softmax_half = [&](int kk) {
#pragma unroll
      for (int qg = 0; qg < QG; ++qg) {
        float e[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          e[j] = fast_exp2(fmaf(sacc[kk][qg][j], p.scale_log2, neg_m[qg]));
          l_run[qg] += e[j];
        }
        pb[kk][0][qg] = pack_bf16x8(e);
        pb[kk][1][qg] = pack_bf16x8(e + 8);
      }
    };
    auto pv_half = [&](int kk) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int tt = 0; tt < NDT; ++tt) {
          const bf16x8_t vf = tr_join(vlo[kk][hh][tt], vhi[kk][hh][tt]);
#pragma unroll
          for (int qg = 0; qg < QG; ++qg)
            oacc[qg][tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[kk][hh][qg], oacc[qg][tt], 0, 0, 0);
        }
    };
    softmax_half(0);
    // Results pass through the waits as operands, so nothing reads them earlier.
    tr_wait_all<NDT>(vlo[0], vhi[0]);
    issue_v(1);
    // The first half's products run on the MFMA pipe while the VALU computes the second half's
    // weights (independent work), one MFMA between every few VALU instructions.
    pv_half(0);
    softmax_half(1);
    {
      constexpr int NM = 2 * NDT * QG, NV = (56 * QG + NM - 1) / NM;
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_VALU, NV, 0);
      }
    }
    tr_wait_all<NDT>(vlo[1], vhi[1]);
    pv_half(1);
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
#pragma unroll 1
  for (int t = 0; t < nt; t += 2) {
    tile(t, S0{});
    if (t + 1 < nt) tile(t + 1, S1{});
  }
#pragma unroll
  for (int qg = 0; qg < QG; ++qg) {
    const float l_tot = l_run[qg] + __shfl_xor(l_run[qg], 32, 64);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qvalid[qg]) {
      bf16_t* O = (bf16_t*)p.O + (int64_t)qrow[qg] * p.ldo + h * D;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const f32x16_t& a = oacc[qg][t];
          *(uint2*)(O + t * 32 + 8 * j4 + 4 * g) = make_uint2(pack2_bf16(a[j4 * 4] * inv, a[j4 * 4 + 1] * inv),
                                                              pack2_bf16(a[j4 * 4 + 2] * inv, a[j4 * 4 + 3] * inv));
        }
      if (g == 0) p.LSE[(int64_t)qrow[qg] * p.Hq + h] = l_tot > 0.f ? m_run[qg] + log2f(l_tot) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Backward: Dsum = rowsum(dO * O) per (row, head); one wavefront per item.
// ---------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void attn_dsum_kernel(const T* __restrict__ dO, int64_t lddo, const T* __restrict__ O,
                                                        int64_t ldo, float* __restrict__ Dsum, int Mq, int Hq, int D) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)Mq * Hq) return;
  const int64_t row = item / Hq;
  const int h = (int)(item % Hq);
  float s = 0.f;
  for (int i = lane; i < D; i += 64)
    s += Elem<T>::load(dO + row * lddo + h * D + i) * Elem<T>::load(O + row * ldo + h * D + i);
  s = wave_sum(s);
  if (lane == 0) Dsum[item] = s;
}

// dQ, bf16: per workgroup 32 NW queries (NW waves x 32) of one head; same tile walk as the
// forward. K and V tiles stream into LDS by buffer loads (two stages). Per 32-key half: S = K Q^T
// and dP = V dO^T, then dS = P (dP - Dsum), then dQ += dS K, whose K^T operand comes from the
// row-major K tile by transpose loads issued before the dS arithmetic.
template <int D, int NW>
__global__ __launch_bounds__(NW * 64, 8 / NW) void attn_dq_bf16_kernel(const AttnArgs p) {
  constexpr int BK = ATT_BK, NKS = D / 16, NDT = D / 32, BQ = 32 * NW;
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];
  bf16_t* Ks = smem;                      // [2][64*D]
  bf16_t* Vs = smem + 2 * BK * D;         // [2][64*D]
  __shared__ int sh[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, lq = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(w);
  const int nqt = (p.Mq + BQ - 1) / BQ;
  const int lin = xcd_remap(blockIdx.x, nqt * p.Hq);
  // K/V-head-major with the heads sharing a K/V head interleaved, as in the forward
  const int rep = p.Hq / p.Hkv, kvh = lin / (nqt * rep), rem = lin % (nqt * rep);
  const int h = kvh * rep + rem % rep, qt = nqt - 1 - rem / rep;
  const int qrow = qt * BQ + w * 32 + lq;
  const bool qvalid = qrow < p.Mq;
  int4 ivq = make_int4(0, 0, 0, 0);
  float lse = 0.f;
  if (qvalid) {
    ivq = *(const int4*)(p.iv + (int64_t)qrow * 8);
    lse = p.LSE[(int64_t)qrow * p.Hq + h];
  }
  // the q-norm backward's per-row scalars, read ahead of the tile walk
  int64_t qkn_ar = 0;
  float qkn_rs = 1.f;
  if (p.qkn_out != nullptr && qvalid) {
    const int64_t pr = p.qkn_pos[qrow];
    qkn_ar = (pr < 0 ? 0 : (pr >= p.qkn_P ? p.qkn_P - 1 : pr)) * (D / 2);
    if (p.qkn_wq) qkn_rs = p.qkn_rstd[(int64_t)qrow * (p.Hq + p.Hkv) + h];
  }
  const bf16_t* Q = (const bf16_t*)p.Q;
  const bf16_t* dO = (const bf16_t*)p.dO;
  const bf16_t* Ob = (const bf16_t*)p.O;
  bf16x8_t qreg[NKS], oreg[NKS];
  // Dsum = rowsum(dO * O) of this (query, head): each lane holds half of the head's dims.
  float dpart = 0.f;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const bf16x8_t z = __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
    qreg[ks] = qvalid ? ld_bf16x8(Q + (int64_t)qrow * p.ldq + h * D + ks * 16 + g * 8) : z;
    oreg[ks] = qvalid ? ld_bf16x8(dO + (int64_t)qrow * p.lddo + h * D + ks * 16 + g * 8) : z;
    const bf16x8_t ov = qvalid ? ld_bf16x8(Ob + (int64_t)qrow * p.ldo + h * D + ks * 16 + g * 8) : z;
#pragma unroll
    for (int e = 0; e < 8; ++e) dpart = fmaf((float)oreg[ks][e], (float)ov[e], dpart);
  }
  const float dsum = dpart + __shfl_xor(dpart, 32, 64);
  if (qvalid && g == 0) p.Dsum[(int64_t)qrow * p.Hq + h] = dsum;
  f32x16_t dq[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[t][r] = 0.f;

  const bool has2 = p.K2 != nullptr;
  Bounds wb1 = wave_bounds(qvalid, ivq.x, ivq.y);
  Bounds wb2 = wave_bounds(has2 && qvalid, ivq.z, ivq.w);
  wb1.lo = __builtin_amdgcn_readfirstlane(wb1.lo); wb1.hi = __builtin_amdgcn_readfirstlane(wb1.hi);
  wb1.maxlo = __builtin_amdgcn_readfirstlane(wb1.maxlo); wb1.minhi = __builtin_amdgcn_readfirstlane(wb1.minhi);
  wb2.lo = __builtin_amdgcn_readfirstlane(wb2.lo); wb2.hi = __builtin_amdgcn_readfirstlane(wb2.hi);
  wb2.maxlo = __builtin_amdgcn_readfirstlane(wb2.maxlo); wb2.minhi = __builtin_amdgcn_readfirstlane(wb2.minhi);
  // workgroup bounds over 8 waves
  if (lane == 0) { sh[w * 2] = wb1.lo; sh[w * 2 + 1] = wb1.hi; }
  __syncthreads();
  int kb1 = INT_MAX, ke1 = INT_MIN;
#pragma unroll
  for (int i = 0; i < NW; ++i) { kb1 = min(kb1, sh[2 * i]); ke1 = max(ke1, sh[2 * i + 1]); }
  __syncthreads();
  if (lane == 0) { sh[w * 2] = wb2.lo; sh[w * 2 + 1] = wb2.hi; }
  __syncthreads();
  int kb2 = INT_MAX, ke2 = INT_MIN;
#pragma unroll
  for (int i = 0; i < NW; ++i) { kb2 = min(kb2, sh[2 * i]); ke2 = max(ke2, sh[2 * i + 1]); }
  kb1 = __builtin_amdgcn_readfirstlane(kb1); ke1 = __builtin_amdgcn_readfirstlane(ke1);
  kb2 = __builtin_amdgcn_readfirstlane(kb2); ke2 = __builtin_amdgcn_readfirstlane(ke2);
  const int n1 = kb1 < ke1 ? (ke1 - (kb1 / BK) * BK + BK - 1) / BK : 0;
  const int n2 = (has2 && kb2 < ke2) ? (ke2 - (kb2 / BK) * BK + BK - 1) / BK : 0;
  const int nt = n1 + n2;

  // Source selection is arithmetic (see the forward kernel).
  const uintptr_t k1a = (uintptr_t)p.K1, v1a = (uintptr_t)p.V1;
  const uintptr_t kd = (uintptr_t)p.K2 - k1a, vd = (uintptr_t)p.V2 - v1a;
  const int64_t ldkd = p.ldk2 - p.ldk1, ldvd = p.ldv2 - p.ldv1;
  const int kt1 = (kb1 / BK) * BK, kt2 = (kb2 / BK) * BK - n1 * BK;
  const uint32_t ko1 = dma_lane_off<D, NW>(p.ldk1, kvh * D, wid, lane);
  const uint32_t vo1 = dma_lane_off<D, NW>(p.ldv1, kvh * D, wid, lane);
  const uint32_t ko2 = has2 ? dma_lane_off<D, NW>(p.ldk2, kvh * D, wid, lane) : 0u;
  const uint32_t vo2 = has2 ? dma_lane_off<D, NW>(p.ldv2, kvh * D, wid, lane) : 0u;
  auto fetch = [&](int t, int stage) {
    const int f2 = t >= n1 ? 1 : 0;
    const int fkt = (f2 ? kt2 : kt1) + t * BK;
    const int fke = ke1 + f2 * (ke2 - ke1);
    dma_tile<D, NW>((const bf16_t*)(k1a + f2 * kd), p.ldk1 + f2 * ldkd, f2 ? ko2 : ko1, fkt, fke, Ks + stage * BK * D, wid);
    dma_tile<D, NW>((const bf16_t*)(v1a + f2 * vd), p.ldv1 + f2 * ldvd, f2 ? vo2 : vo1, fkt, fke, Vs + stage * BK * D, wid);
  };
  // Per-lane LDS offsets, fixed for the whole walk (see the forward kernel).
  int koff[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) koff[ks] = lq * D + (((ks * 2 + g) ^ kswz<D>(lq)) << 3);
  // LDS byte addresses of the K^T transpose loads in stage 0; the stage and the 16-key step are
  // immediate offsets (the tile loop below is unrolled over the two stages).
  uint2 kaddr[NDT];
  const uint32_t kbase0 = lds_addr(Ks);
#pragma unroll
  for (int tt = 0; tt < NDT; ++tt) {
    const int2 o = tr_frag_off<D>(tt, lane);
    kaddr[tt] = make_uint2(kbase0 + 2 * o.x, kbase0 + 2 * o.y);
  }
  if (nt > 0) fetch(0, 0);
  // One K/V tile in LDS stage ST (t & 1), so every stage offset is a compile-time constant.
  auto tile = [&](const int t, auto stc) {
    constexpr int ST = decltype(stc)::value;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();                       // K(t), V(t) in LDS; previous tile's reads are done
    const bf16_t* Kc = Ks + ST * BK * D;
    const bf16_t* Vc = Vs + ST * BK * D;
    if (t + 1 < nt) fetch(t + 1, ST ^ 1);
    const bool s2 = t >= n1;
    const int kt = s2 ? (kb2 / BK) * BK + (t - n1) * BK : (kb1 / BK) * BK + t * BK;
    const int w_lo = s2 ? wb2.lo : wb1.lo, w_hi = s2 ? wb2.hi : wb1.hi;
    const int w_maxlo = s2 ? wb2.maxlo : wb1.maxlo, w_minhi = s2 ? wb2.minhi : wb1.minhi;
    if (kt >= w_hi || kt + BK <= w_lo) return;
    const bool full = kt >= w_maxlo && kt + BK <= w_minhi;
    // key in [lo, hi)  <=>  (unsigned)(key - lo) < (unsigned)(hi - lo)
    const int lo = s2 ? ivq.z : ivq.x;
    const uint32_t span = (uint32_t)max((s2 ? ivq.w : ivq.y) - lo, 0);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      f32x16_t sacc, dpacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) { sacc[r] = 0.f; dpacc[r] = 0.f; }
      // fragments in groups of 4 (16 registers) to stay within two waves per SIMD
#pragma unroll
      for (int k0 = 0; k0 < NKS; k0 += 4) {
        bf16x8_t f[4], v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = *(const bf16x8_t*)(Kc + kk * 32 * D + koff[k0 + i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = *(const bf16x8_t*)(Vc + kk * 32 * D + koff[k0 + i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], qreg[k0 + i], sacc, 0, 0, 0);
          dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v[i], oreg[k0 + i], dpacc, 0, 0, 0);
        }
      }
      // K^T operands of dQ += dS K straight from the row-major K tile (transpose loads): those of
      // the first 16-key step are issued before the dS arithmetic, so that their latency hides
      // behind it, those of the second after it (in flight during the first step's products).
      u32x2_t klo[2][NDT], khi[2][NDT];
      auto issue_k = [&](int hh) {
#pragma unroll
        for (int tt = 0; tt < NDT; ++tt)
          tr_issue_p<D, ST * BK * D * 2>(kaddr[tt], kk * 2 + hh, klo[hh][tt], khi[hh][tt]);
      };
      issue_k(0);
      float pr[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) pr[j] = fast_exp2(fmaf(sacc[j], p.scale_log2, -lse));
      if (!full) {   // wave-uniform: only tiles that cut through some query's interval
        const int d0 = kt + kk * 32 + 4 * g - lo;
#pragma unroll
        for (int j = 0; j < 16; ++j) pr[j] = (uint32_t)(d0 + 8 * (j >> 2) + (j & 3)) < span ? pr[j] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) sacc[j] = pr[j] * (dpacc[j] - dsum);
      bf16x8_t b[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float dv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) dv[i] = sacc[8 * hh + i];
        b[hh] = pack_bf16x8(dv);
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        tr_wait_one<NDT>(klo[hh], khi[hh]);
        if (hh == 0) issue_k(1);
#pragma unroll
        for (int tt = 0; tt < NDT; ++tt)
          dq[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_join(klo[hh][tt], khi[hh][tt]), b[hh], dq[tt], 0, 0, 0);
      }
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
#pragma unroll 1
  for (int t = 0; t < nt; t += 2) {
    tile(t, S0{});
    if (t + 1 < nt) tile(t + 1, S1{});
  }
  if (p.qkn_out != nullptr) {       // wave-uniform: the q/k-norm + RoPE backward on the accumulators
    const int row = qvalid ? qrow : 0;
    qknorm_rope_bwd_acc<D>(dq, p.scale, g, qvalid, p.qkn_pre + (int64_t)row * p.ld_qkn_pre + h * D, qkn_rs, p.qkn_wq,
                           p.qkn_cos + qkn_ar, p.qkn_sin + qkn_ar, p.qkn_out + (int64_t)row * p.ld_qkn_out + h * D);
  } else if (qvalid && p.grad_f32) {
    float* out = (float*)p.dQ + (int64_t)qrow * p.lddq + h * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4)
        *(float4*)(out + t * 32 + 8 * j4 + 4 * g) =
            make_float4(dq[t][j4 * 4] * p.scale, dq[t][j4 * 4 + 1] * p.scale, dq[t][j4 * 4 + 2] * p.scale,
                        dq[t][j4 * 4 + 3] * p.scale);
  } else if (qvalid) {
    bf16_t* out = (bf16_t*)p.dQ + (int64_t)qrow * p.lddq + h * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4)
        *(uint2*)(out + t * 32 + 8 * j4 + 4 * g) =
            make_uint2(pack2_bf16(dq[t][j4 * 4] * p.scale, dq[t][j4 * 4 + 1] * p.scale),
                       pack2_bf16(dq[t][j4 * 4 + 2] * p.scale, dq[t][j4 * 4 + 3] * p.scale));
  }
}

// Rows [q0, q0 + 32) (columns [col0, col0 + D)) of a row-major bf16 matrix into a wave-private
// [32 x D] LDS tile (kswz swizzle) by direct-to-LDS loads issued by one wave; the buffer resource
// covers rows [q0, rend), so rows past rend read as zeros.
template <int D>
__device__ __forceinline__ void dma_rows32(const bf16_t* src, int64_t ld, int col0, int q0, int rend, bf16_t* dst,
                                           int lane) {
  constexpr int CPR = D / 8, RPI = 64 / CPR, INS = 32 / RPI;
  const int rl = lane / CPR, slot = lane % CPR;
  const int nrows = __builtin_amdgcn_readfirstlane(max(0, min(rend - q0, 32)));
  const uintptr_t base = (uintptr_t)(src + (int64_t)q0 * ld + col0);
  const uintptr_t ubase = ((uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32)) << 32) |
                          (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  const int64_t uld = ((int64_t)__builtin_amdgcn_readfirstlane((int)(ld >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)ld);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)ubase, (short)0, (int)((int64_t)nrows * uld * 2), 0x00020000);
#pragma unroll
  for (int i = 0; i < INS; ++i) {
    const int r = i * RPI + rl;
    const uint32_t voff = (uint32_t)r * (uint32_t)uld * 2 + (uint32_t)((slot ^ kswz<D>(r)) << 4);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + i * RPI * D), 16,
                                             voff, 0, 0, 0);
  }
}

// dK, dV of source-2 keys, bf16: per workgroup 128 keys (4 waves x 32) of one kv-head. Each wave
// walks, for every q-head of the GQA group, the 32-query sub-tiles that its keys' query intervals
// [qlo2, qhi2) touch (one per head for blocks up to 32 when the 32 keys fall in aligned blocks),
// staging the Q and dO rows of a sub-tile into its own LDS region (no workgroup barriers).
// Per sub-tile: S = Q K^T and dP = dO V^T with K, V in registers (lane = key), P and dS from
// LSE and Dsum, then dV^T += dO^T P and dK^T += Q^T dS with the transposed operands read from the
// row-major tiles by transpose loads in the accumulator's query order. One workgroup per CU: the
// K, V rows and the dK, dV accumulators need more than the 256 registers of two waves per SIMD,
// and spilling them costs more than the halved occupancy (dK/dV at 4 x 4096, block 16: 109 -> 89 us).
template <int D>
__global__ __launch_bounds__(256, 1) void attn_dkv_bf16_kernel(const AttnArgs p) {
  constexpr int NKS = D / 16, NDT = D / 32, QT = 32;
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];   // per wave: Q [32*D], dO [32*D]
  __shared__ __attribute__((aligned(16))) float s_ld[4][2][QT];     // per wave: LSE, Dsum of the sub-tile
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, lq = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(w);
  bf16_t* Qw = smem + wid * 2 * QT * D;
  bf16_t* Ow = Qw + QT * D;
  const int nkt = (p.Mk2 + 127) / 128;
  const int lin = xcd_remap(blockIdx.x, nkt * p.Hkv);
  const int kvh = lin % p.Hkv, kt = lin / p.Hkv;
  const int rep = p.Hq / p.Hkv;
  const int krow = kt * 128 + w * 32 + lq;
  const bool kvalid = krow < p.Mk2;
  int qlo = 0, qhi = 0;
  if (kvalid) {
    const int2 a = *(const int2*)(p.ivk + (int64_t)krow * 8 + 4);
    qlo = a.x;
    qhi = a.y;
  }
  // query q sees this key  <=>  (unsigned)(q - qlo) < span  (span = 0: no query, or no key)
  const uint32_t span = (uint32_t)max(qhi - qlo, 0);
  // the k-norm backward's per-row scalars, read ahead of the walk
  int64_t qkn_ar = 0;
  float qkn_rs = 1.f;
  if (p.qkn_out != nullptr && kvalid) {
    const int64_t pr = p.qkn_pos[krow];
    qkn_ar = (pr < 0 ? 0 : (pr >= p.qkn_P ? p.qkn_P - 1 : pr)) * (D / 2);
    if (p.qkn_wk) qkn_rs = p.qkn_rstd[(int64_t)krow * (p.Hq + p.Hkv) + p.Hq + kvh];
  }
  const bf16_t* K = (const bf16_t*)p.K2;
  const bf16_t* V = (const bf16_t*)p.V2;
  bf16x8_t kreg[NKS], vreg[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    if (kvalid) {
      kreg[ks] = ld_bf16x8(K + (int64_t)krow * p.ldk2 + kvh * D + ks * 16 + g * 8);
      vreg[ks] = ld_bf16x8(V + (int64_t)krow * p.ldv2 + kvh * D + ks * 16 + g * 8);
    } else {
      kreg[ks] = vreg[ks] = __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
    }
  }
  const int wlo = __builtin_amdgcn_readfirstlane(wave_min_i(span ? qlo : INT_MAX));
  const int whi = __builtin_amdgcn_readfirstlane(wave_max_i(span ? qhi : INT_MIN));
  f32x16_t dk[NDT], dv[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) { dk[t][r] = 0.f; dv[t][r] = 0.f; }
  // Fragment (row lq, chunk 2 ks + g) of a row-major tile sits at lq D + 8 ((2 ks + g) ^ kswz(lq))
  // = kb0 + 16 (ks ^ ksh): two per-lane values instead of NKS offsets.
  const int ksw = kswz<D>(lq);
  const int kb0 = lq * D + 8 * (g ^ (ksw & 1)), ksh = ksw >> 1;
  int2 toff[NDT];
#pragma unroll
  for (int tt = 0; tt < NDT; ++tt) toff[tt] = tr_frag_off<D>(tt, lane);
  const uint32_t qbase = lds_addr(Qw), obase = lds_addr(Ow);
  const bf16_t* Q = (const bf16_t*)p.Q;
  const bf16_t* dO = (const bf16_t*)p.dO;
  if (wlo < whi) {
#pragma unroll 1
    for (int hr = 0; hr < rep; ++hr) {
      const int h = kvh * rep + hr;
#pragma unroll 1
      for (int q0 = (wlo / QT) * QT; q0 < whi; q0 += QT) {
        // The previous sub-tile's LDS reads have all returned (their results fed MFMAs).
        dma_rows32<D>(Q, p.ldq, h * D, q0, p.Mq, Qw, lane);
        dma_rows32<D>(dO, p.lddo, h * D, q0, p.Mq, Ow, lane);
        if (lane < QT) {
          const int qr = q0 + lane;
          const bool ok = qr < p.Mq;
          s_ld[wid][0][lane] = ok ? p.LSE[(int64_t)qr * p.Hq + h] : 0.f;
          s_ld[wid][1][lane] = ok ? p.Dsum[(int64_t)qr * p.Hq + h] : 0.f;
        }
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        f32x16_t sacc, dpacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) { sacc[r] = 0.f; dpacc[r] = 0.f; }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const int off = kb0 + 16 * (ks ^ ksh);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8_t*)(Qw + off), kreg[ks], sacc, 0, 0, 0);
          dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8_t*)(Ow + off), vreg[ks], dpacc, 0, 0, 0);
        }
        // Lane holds queries q0 + 8 (j / 4) + 4 g + (j % 4) of key krow.
        const int dq0 = q0 + 4 * g - qlo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 l4 = *(const float4*)&s_ld[wid][0][8 * i + 4 * g];
          const float4 d4 = *(const float4*)&s_ld[wid][1][8 * i + 4 * g];
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = 4 * i + e;
            const float pe = fast_exp2(fmaf(sacc[j], p.scale_log2, -lv[e]));
            const float pr = (uint32_t)(dq0 + 8 * i + e) < span ? pe : 0.f;
            sacc[j] = pr;
            dpacc[j] = pr * (dpacc[j] - dv4[e]);
          }
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float pv[8], dsv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) { pv[i] = sacc[8 * hh + i]; dsv[i] = dpacc[8 * hh + i]; }
          const bf16x8_t bp = pack_bf16x8(pv), bds = pack_bf16x8(dsv);
          // dO^T and Q^T operands of this 16-query step, two output tiles at a time.
#pragma unroll
          for (int t0 = 0; t0 < NDT; t0 += 2) {
            u32x2_t lo[2][2], hi[2][2];   // [dO, Q][tile]
#pragma unroll
            for (int i = 0; i < 2; ++i) {
              tr_issue_p<D>(make_uint2(obase + 2 * toff[t0 + i].x, obase + 2 * toff[t0 + i].y), hh, lo[0][i], hi[0][i]);
              tr_issue_p<D>(make_uint2(qbase + 2 * toff[t0 + i].x, qbase + 2 * toff[t0 + i].y), hh, lo[1][i], hi[1][i]);
            }
            tr_wait_all<2>(lo, hi);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
              dv[t0 + i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_join(lo[0][i], hi[0][i]), bp, dv[t0 + i], 0, 0, 0);
              dk[t0 + i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_join(lo[1][i], hi[1][i]), bds, dk[t0 + i], 0, 0, 0);
            }
          }
        }
      }
    }
  }
  if (p.qkn_out != nullptr) {       // wave-uniform: the k-norm + RoPE backward on the dK accumulators
    const int row = kvalid ? krow : 0, col = (p.Hq + kvh) * D;
    qknorm_rope_bwd_acc<D>(dk, p.scale, g, kvalid, p.qkn_pre + (int64_t)row * p.ld_qkn_pre + col, qkn_rs, p.qkn_wk,
                           p.qkn_cos + qkn_ar, p.qkn_sin + qkn_ar, p.qkn_out + (int64_t)row * p.ld_qkn_out + col);
  }
  if (kvalid) {
    bf16_t* ov = (bf16_t*)p.dV + (int64_t)krow * p.lddv + kvh * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const int c = t * 32 + 8 * j4 + 4 * g;
        uint2 uv;
        bf16_t* hv = (bf16_t*)&uv;
#pragma unroll
        for (int e = 0; e < 4; ++e) hv[e] = f32_to_bf16(dv[t][j4 * 4 + e]);
        *(uint2*)(ov + c) = uv;
        if (p.qkn_out != nullptr) {
          // dK went through the k-norm backward above
        } else if (p.grad_f32) {
          float* ok = (float*)p.dK + (int64_t)krow * p.lddk + kvh * D;
          *(float4*)(ok + c) = make_float4(dk[t][j4 * 4] * p.scale, dk[t][j4 * 4 + 1] * p.scale,
                                           dk[t][j4 * 4 + 2] * p.scale, dk[t][j4 * 4 + 3] * p.scale);
        } else {
          bf16_t* ok = (bf16_t*)p.dK + (int64_t)krow * p.lddk + kvh * D;
          uint2 uk;
          bf16_t* hk = (bf16_t*)&uk;
#pragma unroll
          for (int e = 0; e < 4; ++e) hk[e] = f32_to_bf16(dk[t][j4 * 4 + e] * p.scale);
          *(uint2*)(ok + c) = uk;
        }
      }
  }
}


// ---------------------------------------------------------------------------------------
// fp32 kernels (fp32 parity mode): one wavefront per (row, head), keys walked one at a time.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_fwd_f32_kernel(const AttnArgs p, int D) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)p.Mq * p.Hq) return;
  const int qrow = (int)(item / p.Hq), h = (int)(item % p.Hq);
  const int kvh = h / (p.Hq / p.Hkv);
  const int4 iv = *(const int4*)(p.iv + (int64_t)qrow * 8);
  const float* q = (const float*)p.Q + (int64_t)qrow * p.ldq + h * D;
  float qv[2] = {0.f, 0.f}, acc[2] = {0.f, 0.f};
  for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) qv[t] = q[lane + 64 * t];
  float m = -INFINITY, l = 0.f;
  for (int src = 0; src < 2; ++src) {
    const float* K = (const float*)(src ? p.K2 : p.K1);
    const float* V = (const float*)(src ? p.V2 : p.V1);
    if (!K) continue;
    const int64_t ldk = src ? p.ldk2 : p.ldk1, ldv = src ? p.ldv2 : p.ldv1;
    const int lo = src ? iv.z : iv.x, hi = src ? iv.w : iv.y;
    for (int k = lo; k < hi; ++k) {
      const float* kr = K + (int64_t)k * ldk + kvh * D;
      float s = 0.f;
      for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) s += qv[t] * kr[lane + 64 * t];
      s = wave_sum(s) * p.scale_log2;
      const float mn = fmaxf(m, s);
      const float a = exp2f(m - mn), e = exp2f(s - mn);
      l = l * a + e;
      const float* vr = V + (int64_t)k * ldv + kvh * D;
      for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) acc[t] = acc[t] * a + e * vr[lane + 64 * t];
      m = mn;
    }
  }
  float* o = (float*)p.O + (int64_t)qrow * p.ldo + h * D;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) o[lane + 64 * t] = acc[t] * inv;
  if (lane == 0) p.LSE[item] = l > 0.f ? m + log2f(l) : -INFINITY;
}

__global__ __launch_bounds__(256) void attn_dq_f32_kernel(const AttnArgs p, int D) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)p.Mq * p.Hq) return;
  const int qrow = (int)(item / p.Hq), h = (int)(item % p.Hq);
  const int kvh = h / (p.Hq / p.Hkv);
  const int4 iv = *(const int4*)(p.iv + (int64_t)qrow * 8);
  const float* q = (const float*)p.Q + (int64_t)qrow * p.ldq + h * D;
  const float* go = (const float*)p.dO + (int64_t)qrow * p.lddo + h * D;
  const float lse = p.LSE[item], ds = p.Dsum[item];
  float qv[2] = {0.f, 0.f}, gv[2] = {0.f, 0.f}, acc[2] = {0.f, 0.f};
  for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) { qv[t] = q[lane + 64 * t]; gv[t] = go[lane + 64 * t]; }
  for (int src = 0; src < 2; ++src) {
    const float* K = (const float*)(src ? p.K2 : p.K1);
    const float* V = (const float*)(src ? p.V2 : p.V1);
    if (!K) continue;
    const int64_t ldk = src ? p.ldk2 : p.ldk1, ldv = src ? p.ldv2 : p.ldv1;
    const int lo = src ? iv.z : iv.x, hi = src ? iv.w : iv.y;
    for (int k = lo; k < hi; ++k) {
      const float* kr = K + (int64_t)k * ldk + kvh * D;
      const float* vr = V + (int64_t)k * ldv + kvh * D;
      float s = 0.f, dp = 0.f;
      for (int t = 0; t < 2; ++t)
        if (lane + 64 * t < D) { s += qv[t] * kr[lane + 64 * t]; dp += gv[t] * vr[lane + 64 * t]; }
      s = wave_sum(s);
      dp = wave_sum(dp);
      const float pr = exp2f(s * p.scale_log2 - lse);
      const float dsc = pr * (dp - ds);
      for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) acc[t] += dsc * kr[lane + 64 * t];
    }
  }
  float* o = (float*)p.dQ + (int64_t)qrow * p.lddq + h * D;
  for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) o[lane + 64 * t] = acc[t] * p.scale;
}

__global__ __launch_bounds__(256) void attn_dkv_f32_kernel(const AttnArgs p, int D) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)p.Mk2 * p.Hkv) return;
  const int krow = (int)(item / p.Hkv), kvh = (int)(item % p.Hkv);
  const int rep = p.Hq / p.Hkv;
  const int qlo = p.ivk[(int64_t)krow * 8 + 4], qhi = p.ivk[(int64_t)krow * 8 + 5];
  const float* kr = (const float*)p.K2 + (int64_t)krow * p.ldk2 + kvh * D;
  const float* vr = (const float*)p.V2 + (int64_t)krow * p.ldv2 + kvh * D;
  float kv[2] = {0.f, 0.f}, vv[2] = {0.f, 0.f}, dk[2] = {0.f, 0.f}, dvv[2] = {0.f, 0.f};
  for (int t = 0; t < 2; ++t) if (lane + 64 * t < D) { kv[t] = kr[lane + 64 * t]; vv[t] = vr[lane + 64 * t]; }
  for (int hr = 0; hr < rep; ++hr) {
    const int h = kvh * rep + hr;
    for (int qr = qlo; qr < qhi; ++qr) {
      const int lo = p.iv[(int64_t)qr * 8 + 2], hi = p.iv[(int64_t)qr * 8 + 3];
      if (krow < lo || krow >= hi) continue;
      const float* q = (const float*)p.Q + (int64_t)qr * p.ldq + h * D;
      const float* go = (const float*)p.dO + (int64_t)qr * p.lddo + h * D;
      float s = 0.f, dp = 0.f;
      for (int t = 0; t < 2; ++t)
        if (lane + 64 * t < D) { s += q[lane + 64 * t] * kv[t]; dp += go[lane + 64 * t] * vv[t]; }
      s = wave_sum(s);
      dp = wave_sum(dp);
      const float pr = exp2f(s * p.scale_log2 - p.LSE[(int64_t)qr * p.Hq + h]);
      const float dsc = pr * (dp - p.Dsum[(int64_t)qr * p.Hq + h]);
      for (int t = 0; t < 2; ++t)
        if (lane + 64 * t < D) { dvv[t] += pr * go[lane + 64 * t]; dk[t] += dsc * q[lane + 64 * t]; }
    }
  }
  float* ok = (float*)p.dK + (int64_t)krow * p.lddk + kvh * D;
  float* ov = (float*)p.dV + (int64_t)krow * p.lddv + kvh * D;
  for (int t = 0; t < 2; ++t)
    if (lane + 64 * t < D) { ok[lane + 64 * t] = dk[t] * p.scale; ov[lane + 64 * t] = dvv[t]; }
}

// ---------------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------------
static int check_geom(int dtype, int D, int Hq, int Hkv) {
  UNOK_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0, UNOK_EINVAL, "attention: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  if (dtype == UNOK_BF16)
    UNOK_REQUIRE(D == 64 || D == 128, UNOK_EUNSUPPORTED, "attention(bf16): head_dim %d not in {64,128}", D);
  else
    UNOK_REQUIRE(D > 0 && D <= 128, UNOK_EUNSUPPORTED, "attention(f32): head_dim %d > 128", D);
  return 0;
}

static bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Forward: 32 queries per wave, 128 per workgroup, two workgroups per CU.
template <int D>
static void launch_fwd(int Mq, int Hq, hipStream_t st, const AttnArgs& a) {
  constexpr size_t lds = 4 * ATT_BK * D * sizeof(bf16_t);
  UNOK_SET_LDS_ONCE((attn_fwd_bf16_kernel<D, 1>), lds);
  const unsigned blocks = (unsigned)(((Mq + 127) / 128) * Hq);
  hipLaunchKernelGGL((attn_fwd_bf16_kernel<D, 1>), dim3(blocks), dim3(256), lds, st, a);
}

// dQ: 4 waves of 32 queries per workgroup, two independent workgroups per CU (their phases
// interleave on each SIMD; with one 8-wave workgroup the two waves of a SIMD pass the same per-tile
// barrier and stall together).
template <int D>
static void launch_dq(int Mq, int Hq, hipStream_t st, const AttnArgs& a) {
  constexpr size_t lds = 4 * ATT_BK * D * sizeof(bf16_t);
  UNOK_SET_LDS_ONCE((attn_dq_bf16_kernel<D, 4>), lds);
  const unsigned blocks = (unsigned)(((Mq + 127) / 128) * Hq);
  hipLaunchKernelGGL((attn_dq_bf16_kernel<D, 4>), dim3(blocks), dim3(256), lds, st, a);
}

template <int D>
static void launch_dkv(unsigned blocks, hipStream_t st, const AttnArgs& a) {
  constexpr size_t lds = 4 * 2 * 32 * D * sizeof(bf16_t);
  UNOK_SET_LDS_ONCE(attn_dkv_bf16_kernel<D>, lds);
  hipLaunchKernelGGL(attn_dkv_bf16_kernel<D>, dim3(blocks), dim3(256), lds, st, a);
}

// Forward. K2/V2 may be null (single source). Strides in elements.
UNOK_EXPORT int unok_attn_fwd(int dtype, int Mq, int Hq, int Hkv, int D, const void* Q, int64_t ldq, const void* K1,
                              int64_t ldk1, const void* V1, int64_t ldv1, const void* K2, int64_t ldk2, const void* V2,
                              int64_t ldv2, const int32_t* iv, void* O, int64_t ldo, float* LSE, float scale,
                              void* stream) {
  if (Mq == 0) return 0;
  int rc = check_geom(dtype, D, Hq, Hkv);
  if (rc) return rc;
  AttnArgs a{};
  a.Q = Q; a.ldq = ldq; a.K1 = K1; a.ldk1 = ldk1; a.V1 = V1; a.ldv1 = ldv1;
  a.K2 = K2; a.ldk2 = ldk2; a.V2 = V2; a.ldv2 = ldv2; a.iv = iv; a.O = O; a.ldo = ldo; a.LSE = LSE;
  a.Mq = Mq; a.Hq = Hq; a.Hkv = Hkv; a.scale = scale; a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == UNOK_F32) {
    hipLaunchKernelGGL(attn_fwd_f32_kernel, dim3((unsigned)(((int64_t)Mq * Hq + 3) / 4)), dim3(256), 0, st, a, D);
  } else {
    UNOK_REQUIRE(dtype == UNOK_BF16, UNOK_EINVAL, "attention: bad dtype %d", dtype);
    UNOK_REQUIRE(al16(Q) && al16(K1) && al16(V1) && ldq % 8 == 0 && ldk1 % 8 == 0 && ldv1 % 8 == 0 && ldo % 8 == 0 &&
                 (!K2 || (al16(K2) && al16(V2) && ldk2 % 8 == 0 && ldv2 % 8 == 0)),
                 UNOK_EALIGN, "attention(bf16): operands must be 16-byte aligned with strides multiple of 8");
    if (D == 128) launch_fwd<128>(Mq, Hq, st, a);
    else launch_fwd<64>(Mq, Hq, st, a);
  }
  return unok::check_launch("attn_fwd");
}

// Split-key forward of decode and draft blocks: S * QR query rows, row i reading query Q[i % QR]
// against one K/V head over its own key interval (the split's share of the cache), with O and
// LSE per row; unok_attn_split_combine merges the S partial rows of each query.
UNOK_EXPORT int unok_attn_fwd_split(int QR, int S, int D, const void* Q, int64_t ldq, const void* K, int64_t ldk,
                                    const void* V, int64_t ldv, const int32_t* iv, void* O, int64_t ldo, float* LSE,
                                    float scale, void* stream) {
  UNOK_REQUIRE(QR >= 0 && S >= 1, UNOK_EINVAL, "attn_fwd_split: QR=%d S=%d", QR, S);
  if (QR == 0) return 0;
  UNOK_REQUIRE((int64_t)QR * S < (1ll << 31), UNOK_EINVAL, "attn_fwd_split: too many rows");
  int rc = check_geom(UNOK_BF16, D, 1, 1);
  if (rc) return rc;
  UNOK_REQUIRE(al16(Q) && al16(K) && al16(V) && al16(O) && ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 &&
                   ldo % 8 == 0,
               UNOK_EALIGN, "attn_fwd_split: operands must be 16-byte aligned with strides multiple of 8");
  AttnArgs a{};
  a.Q = Q; a.ldq = ldq; a.K1 = K; a.ldk1 = ldk; a.V1 = V; a.ldv1 = ldv;
  a.iv = iv; a.O = O; a.ldo = ldo; a.LSE = LSE;
  a.Mq = QR * S; a.Hq = 1; a.Hkv = 1; a.q_mod = QR;
  a.scale = scale; a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) launch_fwd<128>(a.Mq, 1, st, a);
  else launch_fwd<64>(a.Mq, 1, st, a);
  return unok::check_launch("attn_fwd_split");
}

// Backward. Computes Dsum into the caller's [Mq,Hq] fp32 buffer, dQ for every query, and,
// when dK/dV are non-null, dK/dV of the source-2 keys (rows [0, Mk2)). grad_dtype is the element
// type of dQ and dK: dtype, or fp32 with bf16 inputs (dV always has dtype).
UNOK_EXPORT int unok_attn_bwd(int dtype, int grad_dtype, int Mq, int Mk2, int Hq, int Hkv, int D, const void* Q,
                              int64_t ldq,
                              const void* K1, int64_t ldk1, const void* V1, int64_t ldv1, const void* K2, int64_t ldk2,
                              const void* V2, int64_t ldv2, const int32_t* iv, const int32_t* ivk, const void* O,
                              int64_t ldo, const float* LSE, const void* dO, int64_t lddo, float* Dsum, void* dQ,
                              int64_t lddq, void* dK, int64_t lddk, void* dV, int64_t lddv, float scale,
                              void* stream) {
  if (Mq == 0) return 0;
  int rc = check_geom(dtype, D, Hq, Hkv);
  if (rc) return rc;
  UNOK_REQUIRE(grad_dtype == dtype || (dtype == UNOK_BF16 && grad_dtype == UNOK_F32), UNOK_EINVAL,
               "attn_bwd: gradient type %d with input type %d", grad_dtype, dtype);
  hipStream_t st = (hipStream_t)stream;
  const unsigned items = (unsigned)(((int64_t)Mq * Hq + 3) / 4);
  if (dtype == UNOK_F32) {
    // The fp32 path forms Dsum in its own pass; the bf16 dQ kernel forms it on the fly.
    hipLaunchKernelGGL(attn_dsum_kernel<float>, dim3(items), dim3(256), 0, st, (const float*)dO, lddo,
                       (const float*)O, ldo, Dsum, Mq, Hq, D);
    rc = unok::check_launch("attn_dsum");
    if (rc) return rc;
  }
  AttnArgs a{};
  a.O = const_cast<void*>(O); a.ldo = ldo;
  a.Q = Q; a.ldq = ldq; a.K1 = K1; a.ldk1 = ldk1; a.V1 = V1; a.ldv1 = ldv1;
  a.K2 = K2; a.ldk2 = ldk2; a.V2 = V2; a.ldv2 = ldv2; a.iv = iv; a.ivk = ivk; a.LSE = (float*)LSE;
  a.dO = dO; a.lddo = lddo; a.Dsum = Dsum; a.dQ = dQ; a.lddq = lddq; a.dK = dK; a.lddk = lddk; a.dV = dV; a.lddv = lddv;
  a.Mq = Mq; a.Mk2 = Mk2; a.Hq = Hq; a.Hkv = Hkv; a.scale = scale; a.scale_log2 = scale * 1.4426950408889634f;
  a.grad_f32 = dtype == UNOK_BF16 && grad_dtype == UNOK_F32;
  const bool want_kv = dK != nullptr && dV != nullptr && K2 != nullptr && Mk2 > 0;
  if (want_kv) UNOK_REQUIRE(ivk != nullptr, UNOK_EINVAL, "attn_bwd: key-side interval table required for dK/dV");
  if (dtype == UNOK_F32) {
    hipLaunchKernelGGL(attn_dq_f32_kernel, dim3(items), dim3(256), 0, st, a, D);
    rc = unok::check_launch("attn_dq_f32");
    if (rc || !want_kv) return rc;
    hipLaunchKernelGGL(attn_dkv_f32_kernel, dim3((unsigned)(((int64_t)Mk2 * Hkv + 3) / 4)), dim3(256), 0, st, a, D);
    return unok::check_launch("attn_dkv_f32");
  }
  UNOK_REQUIRE(al16(dO) && al16(O) && al16(dQ) && lddo % 8 == 0 && ldo % 8 == 0 && lddq % 8 == 0 &&
                   (!want_kv || (al16(dK) && lddk % 8 == 0 && lddv % 8 == 0)),
               UNOK_EALIGN, "attn_bwd(bf16): gradient strides must be multiples of 8");
  if (D == 128) launch_dq<128>(Mq, Hq, st, a);
  else launch_dq<64>(Mq, Hq, st, a);
  rc = unok::check_launch("attn_dq_bf16");
  if (rc || !want_kv) return rc;
  const unsigned kblocks = (unsigned)(((Mk2 + 127) / 128) * Hkv);
  if (D == 128) launch_dkv<128>(kblocks, st, a);
  else launch_dkv<64>(kblocks, st, a);
  return unok::check_launch("attn_dkv_bf16");
}

// Backward of the noisy stream with the q/k RMSNorm + RoPE backward in the dQ and dK/dV kernels'
// epilogues (bf16): instead of dQ and dK, the gradient before the norm is written into the q and k
// column blocks of dqkv [Mq, (Hq + 2 Hkv) D] (row stride lddqkv), dV into its v block. Source-2
// keys are the query rows themselves (Mk2 = Mq). pre [Mq, (Hq + Hkv) D] holds the pre-norm q/k
// columns (bf16, row stride ldpre), rstd [Mq, Hq + Hkv] their 1/rms (read only with wq / wk),
// cos_tab / sin_tab [P, D/2] the angles at each row's position pos.
UNOK_EXPORT int unok_attn_bwd_qknorm(int Mq, int Hq, int Hkv, int D, const void* Q, int64_t ldq, const void* K1,
                                     int64_t ldk1, const void* V1, int64_t ldv1, const void* K2, int64_t ldk2,
                                     const void* V2, int64_t ldv2, const int32_t* iv, const void* O, int64_t ldo,
                                     const float* LSE, const void* dO, int64_t lddo, float* Dsum, const void* pre,
                                     int64_t ldpre, const float* rstd, const void* wq, const void* wk,
                                     const int64_t* pos, const float* cos_tab, const float* sin_tab, int P,
                                     void* dqkv, int64_t lddqkv, float scale, void* stream) {
  if (Mq == 0) return 0;
  int rc = check_geom(UNOK_BF16, D, Hq, Hkv);
  if (rc) return rc;
  UNOK_REQUIRE(K2 != nullptr && V2 != nullptr && P > 0 && (wq == nullptr) == (wk == nullptr), UNOK_EINVAL,
               "attn_bwd_qknorm: noisy keys, a non-empty angle table and both or neither norm weight required");
  UNOK_REQUIRE(al16(dO) && al16(O) && al16(pre) && al16(dqkv) && al16(cos_tab) && al16(sin_tab) && lddo % 8 == 0 &&
                   ldo % 8 == 0 && ldpre % 8 == 0 && lddqkv % 8 == 0 && (D / 2) % 4 == 0,
               UNOK_EALIGN, "attn_bwd_qknorm: strides must be multiples of 8 and rows 16-byte aligned");
  AttnArgs a{};
  a.O = const_cast<void*>(O); a.ldo = ldo;
  a.Q = Q; a.ldq = ldq; a.K1 = K1; a.ldk1 = ldk1; a.V1 = V1; a.ldv1 = ldv1;
  a.K2 = K2; a.ldk2 = ldk2; a.V2 = V2; a.ldv2 = ldv2; a.iv = iv; a.ivk = iv; a.LSE = (float*)LSE;
  a.dO = dO; a.lddo = lddo; a.Dsum = Dsum;
  a.dV = (bf16_t*)dqkv + (int64_t)(Hq + Hkv) * D; a.lddv = lddqkv;
  a.Mq = Mq; a.Mk2 = Mq; a.Hq = Hq; a.Hkv = Hkv; a.scale = scale; a.scale_log2 = scale * 1.4426950408889634f;
  a.qkn_out = (bf16_t*)dqkv; a.ld_qkn_out = lddqkv;
  a.qkn_pre = (const bf16_t*)pre; a.ld_qkn_pre = ldpre; a.qkn_rstd = rstd;
  a.qkn_wq = (const bf16_t*)wq; a.qkn_wk = (const bf16_t*)wk; a.qkn_pos = pos;
  a.qkn_cos = cos_tab; a.qkn_sin = sin_tab; a.qkn_P = P;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) launch_dq<128>(Mq, Hq, st, a);
  else launch_dq<64>(Mq, Hq, st, a);
  rc = unok::check_launch("attn_dq_bf16");
  if (rc) return rc;
  const unsigned kblocks = (unsigned)(((Mq + 127) / 128) * Hkv);
  if (D == 128) launch_dkv<128>(kblocks, st, a);
  else launch_dkv<64>(kblocks, st, a);
  return unok::check_launch("attn_dkv_bf16");
}
