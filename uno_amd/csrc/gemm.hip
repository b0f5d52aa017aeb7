// GEMM kernels for the conditional-LoRA linears.
//
// All large products of the step are expressed as "NT" GEMMs, C = A * B^T with both operands
// K-contiguous: forward linears use the frozen weight W[out,in]; data gradients use a
// transposed frozen copy W^T[in,out] kept resident in HBM; the LM head uses W_lm[V,H] and
// W_lm^T[H,V]. One MFMA kernel therefore serves every large product.
//
// The LoRA update is fused as a K-extension of the same product:
//   C = alpha * gate (.) ( A[M,K] B[N,K]^T  +  A2[M, col(n) : col(n)+K2] B2[N,K2]^T ) + R
// where, for the forward of a linear, A2 = h = m (.) (x A_lora^T) and B2 = s * B_lora, i.e.
// y = x W^T + s B (m (.) A x) (PEFT LoRA with the token gate, training/lora.py:164-174 and
// peft 0.15.2 lora.Linear.forward). Fused projections (q|k|v, gate|up) carry up to four
// N-segments, each with its own column offset into A2, so the block-diagonal LoRA update
// of a fused projection costs exactly K2 extra K per output column.
//
// The LoRA weight gradients dB = s h^T dY and dA = g^T x are "TN" products (reduction over
// token rows); gemm_tn computes them with split-K partials into a caller workspace.
#include "common.h"
#include "lds_tile.h"

#include <stdlib.h>
#include <type_traits>

struct GemmNT {
  const void* A; int64_t lda;
  const void* B; int64_t ldb;
  const void* A2; int64_t lda2;
  const void* B2; int64_t ldb2;
  void* C; int64_t ldc;
  const void* R; int64_t ldr;
  const uint8_t* gate;
  void* C2; int64_t ldc2;          // second output of the SwiGLU forward epilogue (gate | up), or null
  int group;                       // row tiles per tile group of the 256x256 kernel (0: 8)
  int M, N, K, K2;
  int nseg;
  int seg_end[4];
  int seg_col[4];
  float alpha;
  // LM-head loss epilogues (EPI 3: softmax statistics, EPI 4: cross-entropy gradient) of logits
  // Z = A B^T whose column n is vocabulary entry ce_vocab0 + n.
  const int64_t* ce_tgt;           // [M] target vocabulary ids
  int ce_vocab0;
  float* ce_pmax; float* ce_psum;  // EPI 3: [M, ld ce_ldp] per 128-column block max / sum exp(z - max)
  int64_t ce_ldp;
  float* ce_zt;                    // EPI 3: [M] target logit (rows whose target lies in this product)
  float* ce_z; int64_t ce_ldz;     // EPI 3: [M, ld ce_ldz] the fp32 logits themselves (null: not stored)
  const float* ce_lse;             // EPI 4: [M] log-sum-exp over the whole vocabulary
  const float* ce_w;               // EPI 4: [M] row weights; scaled by *ce_g * *ce_inv_n
  const float* ce_g; const float* ce_inv_n;
  // q|k|v projection epilogue (EPI 5): head dim 128; columns [0, 128 nq) are q heads, then nk k
  // heads, then nk v heads. q/k heads are normalised (when qk_wq is set), scaled by the weight and
  // rotated in fp32, then rounded once into qk_q / qk_k; v heads are rounded into qk_v.
  void* qk_q; void* qk_k; void* qk_v;
  void* qk_pre;                    // [M, 128 (nq+nk)] bf16 q/k before the norm, or null
  float* qk_rstd;                  // [M, nq+nk] 1/rms per row and q/k head, or null
  const void* qk_wq; const void* qk_wk;
  const int64_t* qk_pos;           // [M] position of each row
  const float* qk_cos; const float* qk_sin;   // [qk_P, 64] cos / sin of fl32(position * inv_freq[j])
  int qk_P, qk_nq, qk_nk;
  float qk_eps;
};

template <typename T> __device__ __forceinline__ float ld_f(const T* p);
template <> __device__ __forceinline__ float ld_f<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ld_f<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

// Column offset into A2 of the LoRA segment holding output column n0. Static indexing only, so
// the kernel argument stays in SGPRs (a dynamic index would copy the struct to scratch).
__device__ __forceinline__ int seg_col_of(const GemmNT& p, int n0) {
  int col = p.seg_col[0];
  if (p.nseg > 1 && n0 >= p.seg_end[0]) col = p.seg_col[1];
  if (p.nseg > 2 && n0 >= p.seg_end[1]) col = p.seg_col[2];
  if (p.nseg > 3 && n0 >= p.seg_end[2]) col = p.seg_col[3];
  return col;
}

// ---------------------------------------------------------------------------------------
// bf16 MFMA NT kernel: BM x BN x 64 tiles, 4 waves in a 2x2 grid, each wave computing a
// (BM/2) x (BN/2) sub-tile with v_mfma_f32_32x32x16_bf16. Operand tiles are double
// buffered in LDS (row stride 72 bf16 = 144 B, which makes the 16-byte operand reads of a
// quarter-wave hit distinct banks); the next K tile is fetched into registers while the
// current one is multiplied.
// ---------------------------------------------------------------------------------------
template <int BM, int BN, typename OutT>
__global__ __launch_bounds__(256) void gemm_nt_bf16_kernel(const GemmNT p) {
  constexpr int BK = 64, LDSS = BK + 8;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int ACH = BM * BK / 8 / 256;
  constexpr int BCH = BN * BK / 8 / 256;
  static_assert(ACH >= 1 && BCH >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) bf16_t As[2][BM * LDSS];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][BN * LDSS];

  const int tid = threadIdx.x;
  const int nM = (p.M + BM - 1) / BM, nN = (p.N + BN - 1) / BN;
  const int lin = xcd_remap(blockIdx.x, nM * nN);
  constexpr int GROUP = 8;
  const int group = lin / (GROUP * nN);
  const int first_m = group * GROUP;
  const int gsz = min(nM - first_m, GROUP);
  const int ing = lin % (GROUP * nN);
  const int m0 = (first_m + ing % gsz) * BM;
  const int n0 = (ing / gsz) * BN;

  const bf16_t* A = (const bf16_t*)p.A;
  const bf16_t* B = (const bf16_t*)p.B;
  const bf16_t* A2 = nullptr;
  const bf16_t* B2 = (const bf16_t*)p.B2;
  if (p.A2 != nullptr && p.K2 > 0) A2 = (const bf16_t*)p.A2 + seg_col_of(p, n0);
  const int nk1 = (p.K + BK - 1) / BK;
  const int nk2 = A2 ? (p.K2 + BK - 1) / BK : 0;
  const int nk = nk1 + nk2;

  uint4 ra[ACH], rb[BCH];
  auto load = [&](int kt) {
    const bf16_t* a; const bf16_t* b; int64_t la, lb; int kk, kmax;
    if (kt < nk1) { a = A; b = B; la = p.lda; lb = p.ldb; kk = kt * BK; kmax = p.K; }
    else { a = A2; b = B2; la = p.lda2; lb = p.ldb2; kk = (kt - nk1) * BK; kmax = p.K2; }
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i, r = c >> 3, kc = (c & 7) * 8;
      const int gm = m0 + r, gk = kk + kc;
      ra[i] = (gm < p.M && gk < kmax) ? *(const uint4*)(a + (int64_t)gm * la + gk) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i, r = c >> 3, kc = (c & 7) * 8;
      const int gn = n0 + r, gk = kk + kc;
      rb[i] = (gn < p.N && gk < kmax) ? *(const uint4*)(b + (int64_t)gn * lb + gk) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i, r = c >> 3, kc = (c & 7) * 8;
      *(uint4*)&As[buf][r * LDSS + kc] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i, r = c >> 3, kc = (c & 7) * 8;
      *(uint4*)&Bs[buf][r * LDSS + kc] = rb[i];
    }
  };

  const int lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int lrow = lane & 31, lk = (lane >> 5) * 8;
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *(const bf16x8_t*)&As[buf][(wm * WM + i * 32 + lrow) * LDSS + ks * 16 + lk];
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *(const bf16x8_t*)&Bs[buf][(wn * WN + j * 32 + lrow) * LDSS + ks * 16 + lk];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };

  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load(kt + 1);
    compute(kt & 1);
    if (kt + 1 < nk) store((kt + 1) & 1);
    __syncthreads();
  }

  OutT* C = (OutT*)p.C;
  const OutT* R = (const OutT*)p.R;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * WM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (row >= p.M) continue;
      const bool on = (p.gate == nullptr) || (p.gate[row] != 0);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + lrow;
        if (col >= p.N) continue;
        float v = on ? acc[i][j][r] * p.alpha : 0.f;
        if (R) v += ld_f(R + (int64_t)row * p.ldr + col);
        Elem<OutT>::store(C + (int64_t)row * p.ldc + col, v);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// bf16 MFMA NT kernel with direct global->LDS loads (gfx950 global_load_lds_dwordx4).
// Each lane's 16-byte load lands at LDS base + 16*lane, so one wave instruction fills
// 64*16/(2*BK) consecutive tile rows of BK elements. Rows are stored unpadded; the 16-byte
// chunk c of row r sits at slot c ^ swz(r), chosen so that the 16 lanes one LDS cycle serves
// (rows r0..r0+15 of one chunk column) hit 16 distinct 4-bank groups.
// STAGES LDS buffers form a ring: the loads of K tile kt+STAGES-1 are issued while tile kt is
// multiplied, so STAGES-1 tiles are in flight to cover HBM latency; no VGPR staging and no LDS
// store instructions. One barrier per K tile.
// Requirements (checked on the host): K and K2 multiples of BK, 16-byte aligned operands.
// Rows beyond M (N) are clamped to the last valid row; their results are never stored.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void lds_dma16(const void* g, bf16_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}

template <int BK>
__device__ __forceinline__ int dma_swz(int r) {
  // BK = 64: a row is 32 banks, (r & 1) picks the bank half, the slot picks 4 of its 32 banks.
  // BK = 32: a row is 16 banks, (r & 3) picks the quarter, the slot picks 4 of its 16 banks.
  return BK == 64 ? ((r >> 1) & 7) : ((r >> 2) & 3);
}

template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most `later` (0 .. MAXL, wave-uniform) K tiles of LPT loads each are in flight.
template <int LPT, int MAXL>
__device__ __forceinline__ void wait_tiles(int later) {
  if constexpr (MAXL == 0) {
    wait_vm<0>();
  } else {
    if (later >= MAXL) wait_vm<MAXL * LPT>();
    else wait_tiles<LPT, MAXL - 1>(later);
  }
}

template <int BM, int BN, int NW, int BK, int STAGES, typename OutT, bool ROT = false>
__global__ __launch_bounds__(NW * 64) void gemm_nt_bf16_dma_kernel(const GemmNT p) {
  constexpr int CPR = BK / 8;                     // 16-byte chunks per tile row
  constexpr int RPI = 64 / CPR;                   // tile rows per wave load instruction
  constexpr int WAVES_N = 2, WAVES_M = NW / WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_INS = BM / (RPI * NW), B_INS = BN / (RPI * NW);   // load instructions per wave
  constexpr int LPT = A_INS + B_INS;              // loads per wave per K tile
  static_assert(A_INS >= 1 && B_INS >= 1 && TM >= 1 && TN >= 1, "bad tile");
  static_assert(STAGES >= 2 && (STAGES - 2) * LPT < 64, "bad stage count");
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];
  bf16_t* As = smem;                              // [STAGES][BM*BK]
  bf16_t* Bs = smem + STAGES * BM * BK;           // [STAGES][BN*BK]

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nM = (p.M + BM - 1) / BM, nN = (p.N + BN - 1) / BN;
  const int lin = xcd_remap(blockIdx.x, nM * nN);
  constexpr int GROUP = 8;
  const int group = lin / (GROUP * nN);
  const int first_m = group * GROUP;
  const int gsz = min(nM - first_m, GROUP);
  const int ing = lin % (GROUP * nN);
  const int m0 = (first_m + ing % gsz) * BM;
  const int n0 = (ing / gsz) * BN;

  const bf16_t* A = (const bf16_t*)p.A;
  const bf16_t* B = (const bf16_t*)p.B;
  const bf16_t* A2 = nullptr;
  if (p.A2 != nullptr && p.K2 > 0) A2 = (const bf16_t*)p.A2 + seg_col_of(p, n0);
  const bf16_t* B2 = (const bf16_t*)p.B2;
  const int nk1 = p.K / BK;
  const int nk = nk1 + (A2 ? p.K2 / BK : 0);

  // Per-lane source rows (clamped) and swizzled chunk, fixed for the whole K loop.
  const int lrowi = lane / CPR, slot = lane % CPR;
  int64_t a_off[A_INS], b_off[B_INS], a2_off[A_INS], b2_off[B_INS];
#pragma unroll
  for (int i = 0; i < A_INS; ++i) {
    const int r = (i * NW + wid) * RPI + lrowi;
    const int gm = min(m0 + r, p.M - 1);
    const int chunk = slot ^ dma_swz<BK>(r);
    a_off[i] = (int64_t)gm * p.lda + chunk * 8;
    a2_off[i] = (int64_t)gm * p.lda2 + chunk * 8;
  }
#pragma unroll
  for (int i = 0; i < B_INS; ++i) {
    const int r = (i * NW + wid) * RPI + lrowi;
    const int gn = min(n0 + r, p.N - 1);
    const int chunk = slot ^ dma_swz<BK>(r);
    b_off[i] = (int64_t)gn * p.ldb + chunk * 8;
    b2_off[i] = (int64_t)gn * p.ldb2 + chunk * 8;
  }
  // With ROT, workgroup b walks the main K tiles starting at tile (7 b) mod nk1: workgroups that
  // run at the same time then read different column offsets of their rows instead of the same one.
  const int rot = ROT && nk1 > 0 ? (int)((7u * blockIdx.x) % (unsigned)nk1) : 0;
  auto issue = [&](int kt, int buf) {
    bf16_t* as = As + buf * BM * BK;
    bf16_t* bs = Bs + buf * BN * BK;
    if (kt < nk1) {
      const int kr = kt + rot;
      const int kk = (kr >= nk1 ? kr - nk1 : kr) * BK;
#pragma unroll
      for (int i = 0; i < A_INS; ++i) lds_dma16(A + a_off[i] + kk, as + (i * NW + wid) * RPI * BK);
#pragma unroll
      for (int i = 0; i < B_INS; ++i) lds_dma16(B + b_off[i] + kk, bs + (i * NW + wid) * RPI * BK);
    } else {
      const int kk = (kt - nk1) * BK;
#pragma unroll
      for (int i = 0; i < A_INS; ++i) lds_dma16(A2 + a2_off[i] + kk, as + (i * NW + wid) * RPI * BK);
#pragma unroll
      for (int i = 0; i < B_INS; ++i) lds_dma16(B2 + b2_off[i] + kk, bs + (i * NW + wid) * RPI * BK);
    }
  };

  const int wm = wid / WAVES_N, wn = wid % WAVES_N;
  const int lrow = lane & 31, lg = lane >> 5;
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto compute = [&](int buf) {
    const bf16_t* as = As + buf * BM * BK;
    const bf16_t* bs = Bs + buf * BN * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = ks * 2 + lg;
      bf16x8_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + i * 32 + lrow;
        a[i] = *(const bf16x8_t*)&as[r * BK + ((chunk ^ dma_swz<BK>(r)) << 3)];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WN + j * 32 + lrow;
        b[j] = *(const bf16x8_t*)&bs[r * BK + ((chunk ^ dma_swz<BK>(r)) << 3)];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) issue(s, s);
  for (int kt = 0; kt < nk; ++kt) {
    // Tile kt has landed once at most (tiles issued after it) * LPT loads are outstanding.
    wait_tiles<LPT, STAGES - 2>(min(nk - 1 - kt, STAGES - 2));
    // Plain s_barrier: a __syncthreads() fence would also wait for the tiles still in flight.
    // Each wave has waited for its own loads of tile kt above, so after the barrier the whole
    // tile is in LDS; the "memory" clobber keeps the compiler from moving LDS reads across it.
    asm volatile("s_barrier" ::: "memory");
    if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
    compute(kt % STAGES);
  }

  OutT* C = (OutT*)p.C;
  const OutT* R = (const OutT*)p.R;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * WM + i * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
      if (row >= p.M) continue;
      const bool on = (p.gate == nullptr) || (p.gate[row] != 0);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + lrow;
        if (col >= p.N) continue;
        float v = on ? acc[i][j][r] * p.alpha : 0.f;
        if (R) v += ld_f(R + (int64_t)row * p.ldr + col);
        Elem<OutT>::store(C + (int64_t)row * p.ldc + col, v);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Helpers of the 256x256 direct-to-LDS kernel below: buffer resources and 4-wide epilogue stores.
// ---------------------------------------------------------------------------------------
// Buffer resource over `bytes` bytes from `base` (raw buffer: stride 0, dword 3 = data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void buf_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, bf16_t* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// dst[0..3] = v[0..3] (+ res[0..3]) as one vector store (8 bytes for bf16, 16 for fp32).
__device__ __forceinline__ void store4(bf16_t* dst, const bf16_t* res, const float (&v)[4]) {
  float a0 = v[0], a1 = v[1], a2 = v[2], a3 = v[3];
  if (res) {
    const uint2 r = *(const uint2*)res;
    a0 += __uint_as_float(r.x << 16); a1 += __uint_as_float(r.x & 0xffff0000u);
    a2 += __uint_as_float(r.y << 16); a3 += __uint_as_float(r.y & 0xffff0000u);
  }
  *(uint2*)dst = make_uint2(pack2_bf16(a0, a1), pack2_bf16(a2, a3));
}
__device__ __forceinline__ void store4(float* dst, const float* res, const float (&v)[4]) {
  float4 o = make_float4(v[0], v[1], v[2], v[3]);
  if (res) {
    const float4 r = *(const float4*)res;
    o.x += r.x; o.y += r.y; o.z += r.z; o.w += r.w;
  }
  *(float4*)dst = o;
}

// ---------------------------------------------------------------------------------------
// fp32 NT kernel (fp32 parity mode): 64x64 tiles, 16-deep K slices, 4x4 outputs per thread.
// ---------------------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(256) void gemm_nt_f32_kernel(const GemmNT p) {
  __shared__ float As[16][65], Bs[16][65];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const float* A = (const float*)p.A;
  const float* B = (const float*)p.B;
  const float* A2 = nullptr;
  if (p.A2 != nullptr && p.K2 > 0) A2 = (const float*)p.A2 + seg_col_of(p, n0);
  const float* B2 = (const float*)p.B2;
  float acc[4][4] = {};
  for (int part = 0; part < 2; ++part) {
    const float* a = part ? A2 : A;
    const float* b = part ? B2 : B;
    if (a == nullptr) continue;
    const int64_t la = part ? p.lda2 : p.lda, lb = part ? p.ldb2 : p.ldb;
    const int K = part ? p.K2 : p.K;
    for (int k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = tid + 256 * q, r = e >> 4, k = e & 15;
        const int gm = m0 + r, gn = n0 + r, gk = k0 + k;
        As[k][r] = (gm < p.M && gk < K) ? a[(int64_t)gm * la + gk] : 0.f;
        Bs[k][r] = (gn < p.N && gk < K) ? b[(int64_t)gn * lb + gk] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        float av[4], bv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) av[i] = As[k][ty + 16 * i];
#pragma unroll
        for (int j = 0; j < 4; ++j) bv[j] = Bs[k][tx + 16 * j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
      }
      __syncthreads();
    }
  }
  OutT* C = (OutT*)p.C;
  const OutT* R = (const OutT*)p.R;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + ty + 16 * i;
    if (row >= p.M) continue;
    const bool on = (p.gate == nullptr) || (p.gate[row] != 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + tx + 16 * j;
      if (col >= p.N) continue;
      float v = on ? acc[i][j] * p.alpha : 0.f;
      if (R) v += ld_f(R + (int64_t)row * p.ldr + col);
      Elem<OutT>::store(C + (int64_t)row * p.ldc + col, v);
    }
  }
}

// ---------------------------------------------------------------------------------------
// TN products for LoRA weight gradients: WS[z][P][Q] = alpha * sum_{m in split z} A[m,p] B[m,q].
// The bf16 kernel stages A^T and B^T tiles in LDS (transposing 16-byte global loads into
// m-contiguous rows) and then runs the same MFMA inner loop as the NT kernel.
// ---------------------------------------------------------------------------------------
struct GemmTN {
  const void* A; int64_t lda;   // [Mrows, P]
  const void* B; int64_t ldb;   // [Mrows, Q]
  float* WS;                     // [nsplit, P, Q]
  int Mrows, P, Q, rows_per_split;
  float alpha;
};

template <int BP, int BQ>
__global__ __launch_bounds__(256) void gemm_tn_bf16_kernel(const GemmTN p) {
  constexpr int BK = 64, LDSS = BK + 8;
  constexpr int WP = BP / 2, WQ = BQ / 2;
  constexpr int TM = WP / 32, TN = WQ / 32;
  constexpr int ACH = BP * BK / 8 / 256;
  constexpr int BCH = BQ * BK / 8 / 256;
  __shared__ __attribute__((aligned(16))) bf16_t As[BP * LDSS];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[BQ * LDSS];
  const int tid = threadIdx.x;
  const int nQ = (p.Q + BQ - 1) / BQ;
  const int p0 = (blockIdx.x / nQ) * BP, q0 = (blockIdx.x % nQ) * BQ;
  const int mbeg = blockIdx.y * p.rows_per_split;
  const int mend = min(p.Mrows, mbeg + p.rows_per_split);
  const bf16_t* A = (const bf16_t*)p.A;
  const bf16_t* B = (const bf16_t*)p.B;
  const int lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int lrow = lane & 31, lk = (lane >> 5) * 8;
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  for (int mk = mbeg; mk < mend; mk += BK) {
    uint4 ra[ACH], rb[BCH];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i, r = c / (BP / 8), pc = (c % (BP / 8)) * 8;
      const int gm = mk + r, gp = p0 + pc;
      ra[i] = (gm < mend && gp < p.P) ? *(const uint4*)(A + (int64_t)gm * p.lda + gp) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i, r = c / (BQ / 8), qc = (c % (BQ / 8)) * 8;
      const int gm = mk + r, gq = q0 + qc;
      rb[i] = (gm < mend && gq < p.Q) ? *(const uint4*)(B + (int64_t)gm * p.ldb + gq) : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i, r = c / (BP / 8), pc = (c % (BP / 8)) * 8;
      const bf16_t* v = (const bf16_t*)&ra[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) As[(pc + e) * LDSS + r] = v[e];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i, r = c / (BQ / 8), qc = (c % (BQ / 8)) * 8;
      const bf16_t* v = (const bf16_t*)&rb[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) Bs[(qc + e) * LDSS + r] = v[e];
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const bf16x8_t*)&As[(wm * WP + i * 32 + lrow) * LDSS + ks * 16 + lk];
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const bf16x8_t*)&Bs[(wn * WQ + j * 32 + lrow) * LDSS + ks * 16 + lk];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }
  float* W = p.WS + (int64_t)blockIdx.y * p.P * p.Q;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = p0 + wm * WP + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (row >= p.P) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = q0 + wn * WQ + j * 32 + lrow;
        if (col < p.Q) W[(int64_t)row * p.Q + col] = acc[i][j][r] * p.alpha;
      }
    }
}

__global__ __launch_bounds__(256) void gemm_tn_f32_kernel(const GemmTN p) {
  __shared__ float As[16][65], Bs[16][65];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int nQ = (p.Q + 63) / 64;
  const int p0 = (blockIdx.x / nQ) * 64, q0 = (blockIdx.x % nQ) * 64;
  const int mbeg = blockIdx.y * p.rows_per_split;
  const int mend = min(p.Mrows, mbeg + p.rows_per_split);
  const float* A = (const float*)p.A;
  const float* B = (const float*)p.B;
  float acc[4][4] = {};
  for (int mk = mbeg; mk < mend; mk += 16) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = tid + 256 * q, k = e >> 6, c = e & 63;
      const int gm = mk + k;
      As[k][c] = (gm < mend && p0 + c < p.P) ? A[(int64_t)gm * p.lda + p0 + c] : 0.f;
      Bs[k][c] = (gm < mend && q0 + c < p.Q) ? B[(int64_t)gm * p.ldb + q0 + c] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[k][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[k][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
  float* W = p.WS + (int64_t)blockIdx.y * p.P * p.Q;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = p0 + ty + 16 * i;
    if (row >= p.P) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = q0 + tx + 16 * j;
      if (col < p.Q) W[(int64_t)row * p.Q + col] = acc[i][j] * p.alpha;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Skinny TN product of the LoRA weight gradients:
//   WS[z][s][x] = alpha * sum_{m in rows of split z} S[m, s] X[m, x]
// S is the rank-side operand (g or h: 32 .. 192 columns in steps of 32, or 256 / 384) and X the
// wide activation or gradient (x, dY). The product is HBM-bound on X, so X is streamed once: a
// workgroup owns a strip of X columns and a contiguous range of token rows (a split); the splits'
// fp32 partials are added by splitk_reduce_kernel. The kernels are gemm_tn_tr_kernel and
// gemm_tn_trw_kernel below, next to the C-ABI.
// ---------------------------------------------------------------------------------------
struct GemmTNSkinny {
  const bf16_t* S; int64_t lds;   // [Mrows, NS]
  const bf16_t* X; int64_t ldx;   // [Mrows, NX]
  float* WS;                       // [nsplit, NS, NX] or, transposed, [nsplit, NX, NS]
  int Mrows, NS, NX, rows_per_split;
  float alpha;
};

constexpr int TNS_MIN_NX = 256;   // narrowest wide side the skinny path takes
constexpr int TNS_BK = 64;        // token rows per tile (split ranges are whole tiles)

// C[P,Q] (row stride ldc, fp32) = beta * C + sum_z WS[z], partials summed in z order. With Q and
// ldc multiples of 4 and 16-byte aligned buffers each thread takes 4 consecutive elements, and
// the partial loads are unrolled so several are in flight at once.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, float* C, int64_t ldc,
                                                             int P, int Q, int nsplit, float beta) {
  const int64_t total = (int64_t)P * Q;
  const bool vec = (Q & 3) == 0 && (ldc & 3) == 0 && (((uintptr_t)ws | (uintptr_t)C) & 15) == 0;
  if (vec) {
    for (int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x); i < total;
         i += 4 * (int64_t)gridDim.x * blockDim.x) {
      float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
      for (int z = 0; z < nsplit; ++z) {
        const float4 v = *(const float4*)(ws + z * total + i);
        s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
      }
      const int64_t r = i / Q, c = i % Q;
      float4* dst = (float4*)(C + r * ldc + c);
      if (beta != 0.f) {
        const float4 o = *dst;
        s.x += beta * o.x; s.y += beta * o.y; s.z += beta * o.z; s.w += beta * o.w;
      }
      *dst = s;
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
#pragma unroll 4
    for (int z = 0; z < nsplit; ++z) s += ws[z * total + i];
    const int64_t r = i / Q, c = i % Q;
    float* dst = C + r * ldc + c;
    *dst = (beta != 0.f ? beta * *dst : 0.f) + s;
  }
}

// Workgroups of the split-K reduction: one element per thread, four when rows allow vectors.
static int reduce_blocks(int P, int Q) {
  const int64_t per = (Q % 4 == 0) ? 1024 : 256;
  const int64_t b = ((int64_t)P * Q + per - 1) / per;
  return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

// ---------------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------------
template <int BM, int BN>
static void launch_nt_bf16(const GemmNT& p, int out_dtype, hipStream_t st) {
  const int nb = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  if (out_dtype == UNOK_BF16)
    hipLaunchKernelGGL((gemm_nt_bf16_kernel<BM, BN, bf16_t>), dim3(nb), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_nt_bf16_kernel<BM, BN, float>), dim3(nb), dim3(256), 0, st, p);
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// ---------------------------------------------------------------------------------------
// 256x256 bf16 NT kernel with 16x16x32 MFMAs: 4 waves of 128x128 (8 x 8 accumulators of 4 floats,
// 256 AGPRs), BK 64, A tiles in 3 LDS stages and B tiles in 2 (160 KB), filled by direct-to-LDS
// loads with the same swizzled layout as the 32x32x16 kernel. A tile is two 32-wide k-steps: step 0
// reads step 1's fragments and issues the A loads of the tile two ahead, then the barrier, then
// step 1 reads the next tile's step-0 fragments and issues that tile's B loads (one load per eight
// MFMAs in both steps: with all 16 in one step the 64 B/clk vector-memory path saturated and
// stalled the MFMA stream). Per 32 k and wave: 8 A + 8 B fragment reads (16 bytes per lane) and 64
// MFMAs. With the B fragment as the first operand, lane l holds C[row 16i + l % 16][cols 16j +
// 4 (l / 16) + 0..3] of accumulator (i, j).
// ---------------------------------------------------------------------------------------
template <typename OutT, int EPI = 0>
__global__ __launch_bounds__(256) void gemm_nt_bf16_w4m16_kernel(const GemmNT p) {
  constexpr int BM = 256, BN = 256, BK = 64, NW = 4, TM = 8, TN = 8;
  constexpr int CPR = BK / 8, RPI = 64 / CPR, INS = BM / (RPI * NW);   // 8 loads per operand and wave
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];
  bf16_t* As = smem;                            // [3][BM*BK]
  bf16_t* Bs = smem + 3 * BM * BK;              // [2][BN*BK]

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nM = (p.M + BM - 1) / BM, nN = (p.N + BN - 1) / BN;
  const int lin = xcd_remap(blockIdx.x, nM * nN);
  const int GROUP = p.group > 0 ? p.group : 8;
  const int group = lin / (GROUP * nN);
  const int first_m = group * GROUP;
  const int gsz = min(nM - first_m, GROUP);
  const int ing = lin % (GROUP * nN);
  const int m0 = (first_m + ing % gsz) * BM;
  const int n0 = (ing / gsz) * BN;
  const bool ext = p.A2 != nullptr && p.K2 > 0;
  const int nk1 = p.K / BK;
  // The LoRA extension runs in whole 64-deep tiles; K2 = 32 (mod 64) leaves the last one half full,
  // and its second 32-wide k-step then runs on zeroed fragments.
  const int nk = nk1 + (ext ? (p.K2 + BK - 1) / BK : 0);
  const bool half_last = ext && (p.K2 % BK) != 0;

  const int lrowi = lane / CPR, slot = lane % CPR;
  // Operand rows are addressed from this tile's first row, so the 32-bit buffer offsets span one
  // 256-row strip rather than the whole operand (rows past the end clamp to its last row).
  const int mrows = min(p.M - m0, BM), nrows = min(p.N - n0, BN);
  __amdgpu_buffer_rsrc_t ra = make_rsrc((const bf16_t*)p.A + (int64_t)m0 * p.lda,
                                        (uint32_t)(((int64_t)(mrows - 1) * p.lda + p.K) * 2));
  __amdgpu_buffer_rsrc_t rb = make_rsrc((const bf16_t*)p.B + (int64_t)n0 * p.ldb,
                                        (uint32_t)(((int64_t)(nrows - 1) * p.ldb + p.K) * 2));
  uint32_t a_vo[INS], b_vo[INS];
  auto set_offsets = [&](int64_t lda, int64_t ldb) {
#pragma unroll
    for (int i = 0; i < INS; ++i) {
      const int r = (i * NW + wid) * RPI + lrowi;
      const int chunk = slot ^ dma_swz<BK>(r);
      a_vo[i] = (uint32_t)(((int64_t)min(r, mrows - 1) * lda + chunk * 8) * 2);
      b_vo[i] = (uint32_t)(((int64_t)min(r, nrows - 1) * ldb + chunk * 8) * 2);
    }
  };
  set_offsets(p.lda, p.ldb);
  int kbase = 0;
  // Sets up the operand pair of tile t (the LoRA pair from tile nk1 on; tiles are set up in
  // order) and returns its k byte offset.
  auto dma_tile = [&](int t) -> uint32_t {
    if (t == nk1) {
      ra = make_rsrc((const bf16_t*)p.A2 + seg_col_of(p, n0) + (int64_t)m0 * p.lda2,
                     (uint32_t)(((int64_t)(mrows - 1) * p.lda2 + p.K2) * 2));
      rb = make_rsrc((const bf16_t*)p.B2 + (int64_t)n0 * p.ldb2, (uint32_t)(((int64_t)(nrows - 1) * p.ldb2 + p.K2) * 2));
      set_offsets(p.lda2, p.ldb2);
      kbase = nk1;
    }
    return (uint32_t)(t - kbase) * BK * 2;
  };
  auto dma_one = [&](int n, uint32_t kb, int stage) {
    bf16_t* as = As + stage * BM * BK + wid * RPI * BK;
    bf16_t* bs = Bs + stage * BN * BK + wid * RPI * BK;
    if (n < INS) buf_lds16(ra, a_vo[n], kb, as + n * NW * RPI * BK);
    else buf_lds16(rb, b_vo[n - INS], kb, bs + (n - INS) * NW * RPI * BK);
  };

  // Fragment rows wm*128 + 16i + lane%16 (A) / wn*128 + 16j + lane%16 (B); chunk 4s + lane/16 of
  // the 8 in a row (k-step s); every such row has the swizzle dma_swz(lane % 16).
  const int wm = wid >> 1, wn = wid & 1;
  const int lr = lane & 15, lk = lane >> 4;
  const int sw = dma_swz<BK>(lr);
  const int a_row0 = (wm * 128 + lr) * BK, b_row0 = (wn * 128 + lr) * BK;
  bf16x8_t fa0[TM], fb0[TN], fa1[TM], fb1[TN];

  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

  // One k-step: 64 MFMAs on (fa, fb); after every fourth a fragment read of A stage ra_st / B
  // stage rb_st, k-step rs, in the order the next step consumes them (fa[0], fb[0..7], fa[1..7]);
  // between two of those reads, after every eighth MFMA (the third of each eight), one of the 8
  // direct-to-LDS loads of operand LB (0: A, 1: B) into stage dst.
  auto step = [&](const bf16x8_t (&fa)[TM], const bf16x8_t (&fb)[TN], bf16x8_t (&na)[TM], bf16x8_t (&nb)[TN],
                  int ra_st, int rb_st, int rs, auto lb, uint32_t kb, int dst) {
    constexpr int LB = decltype(lb)::value;
    const bf16_t* as = As + ra_st * BM * BK + a_row0;
    const bf16_t* bs = Bs + rb_st * BN * BK + b_row0;
    const int co = ((4 * rs + lk) ^ sw) << 3;
#pragma unroll
    for (int idx = 0; idx < TM * TN; ++idx) {
      const int i = idx / TN, j = idx % TN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
      if (idx % 8 == 2) dma_one(LB * INS + idx / 8, kb, dst);
      if (idx % 4 == 0) {
        const int r = idx / 4;   // 0: fa[0]; 1..8: fb[0..7]; 9..15: fa[1..7]
        if (r == 0) na[0] = *(const bf16x8_t*)&as[co];
        else if (r <= TN) nb[r - 1] = *(const bf16x8_t*)&bs[(r - 1) * 16 * BK + co];
        else na[r - TN] = *(const bf16x8_t*)&as[(r - TN) * 16 * BK + co];
      }
    }
#pragma unroll
    for (int idx = 0; idx < TM * TN; ++idx) {
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
      if (idx % 8 == 2) __builtin_amdgcn_sched_group_barrier(SG_VMEM, 1, 0);
      if (idx % 4 == 0) __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  using LA = std::integral_constant<int, 0>;
  using LBt = std::integral_constant<int, 1>;

  // Prologue: tiles 0 and 1 (clamped) in full; wait for tile 0; its step-0 fragments.
  {
    uint32_t kb = dma_tile(0);
#pragma unroll
    for (int n = 0; n < 2 * INS; ++n) dma_one(n, kb, 0);
    kb = dma_tile(min(1, nk - 1));
#pragma unroll
    for (int n = 0; n < 2 * INS; ++n) dma_one(n, kb, 1);
  }
  wait_vm<2 * INS>();
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("s_barrier" ::: "memory");
  {
    const bf16_t* as = As + a_row0;
    const bf16_t* bs = Bs + b_row0;
    const int co = (lk ^ sw) << 3;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa0[i] = *(const bf16x8_t*)&as[i * 16 * BK + co];
#pragma unroll
    for (int j = 0; j < TN; ++j) fb0[j] = *(const bf16x8_t*)&bs[j * 16 * BK + co];
  }
  // A tiles rotate through 3 stages, B tiles through 2. Tile kt+2's A loads fly during tile kt's
  // first step (into the A stage tile kt-1 used, free since tile kt-1's middle barrier), its B
  // loads during the second (into tile kt's B stage, free after this tile's middle barrier), so
  // every step carries 8 loads per wave and the A loads have two to three steps to land.
  int sa = 0;                 // A stage of tile kt
  for (int kt = 0; kt < nk; ++kt) {
    const int sa1 = sa == 2 ? 0 : sa + 1, sa2 = sa1 == 2 ? 0 : sa1 + 1;
    const int sb = kt & 1;
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t kb = dma_tile(min(kt + 2, nk - 1));
    step(fa0, fb0, fa1, fb1, sa, sb, 1, LA{}, kb, sa2);
    // Tile kt+1 is complete once every wave is here with its loads landed (only tile kt+2's A
    // loads may still fly); tile kt's B stage is free.
    wait_vm<INS>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (half_last && kt == nk - 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i) fa1[i] = __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
#pragma unroll
      for (int j = 0; j < TN; ++j) fb1[j] = __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
    }
    step(fa1, fb1, fa0, fb0, sa1, sb ^ 1, 0, LBt{}, kb, sb);
    sa = sa1;
  }
  __builtin_amdgcn_s_waitcnt(0x0070);       // clamped loads still write LDS

  OutT* C = (OutT*)p.C;
  const OutT* R = (const OutT*)p.R;
  auto epilogue = [&](auto has_res, auto checked) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm * 128 + i * 16 + lr;
      if (checked && row >= p.M) continue;
      const float sc = (!checked || p.gate == nullptr || p.gate[row] != 0) ? p.alpha : 0.f;
      OutT* crow = C + (int64_t)row * p.ldc;
      const OutT* rrow = has_res ? R + (int64_t)row * p.ldr : nullptr;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * 128 + j * 16 + lk * 4;
        if (checked && col >= p.N) continue;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = acc[i][j][q] * sc;
        store4(crow + col, has_res ? rrow + col : nullptr, v);
      }
    }
  };
  if constexpr (EPI == 2) {
    // SwiGLU backward of the down-projection data gradient: this product is dS[M, F] (never
    // stored); with R = gu [M, 2F] (ldr) and C = dgu [M, 2F] (ldc), writes dgu[:, f] and
    // dgu[:, F + f] from bf16(dS), g = gu[:, f], u = gu[:, F + f], as the SwiGLU backward kernel
    // does after a bf16 product. Interior tiles only (checked by the caller). Each wave rounds its
    // 128 x 128 quadrant of dS into a private 32 KB of the (now idle) LDS stages, 16-byte chunks
    // XOR-swizzled by row so that both the fragment-ordered writes and the row-ordered reads are
    // conflict-free, then walks it four rows per step: every gu load and dgu store is a 256-byte
    // run per row (16 bytes per lane), with the gu loads of the next DEPTH batches of eight rows
    // in flight (the K loop's fragment registers hold them), the first ones issued before the
    // staging so that their latency passes behind it.
    constexpr int PB = 2, NBATCH = 128 / (4 * PB), DEPTH = 6;
    const int F = p.N;
    const int rsub = lane >> 4, c16 = lane & 15;
    const int64_t row0 = m0 + wm * 128 + rsub;
    const int col = n0 + wn * 128 + c16 * 8;
    const bf16_t* gsrc = (const bf16_t*)p.R + row0 * p.ldr + col;
    bf16_t* dst = (bf16_t*)p.C + row0 * p.ldc + col;
    uint4 gw[NBATCH][PB], uw[NBATCH][PB];   // fully unrolled: only DEPTH + 1 batches are live
    auto load_batch = [&](int b) {
#pragma unroll
      for (int t = 0; t < PB; ++t) {
        const bf16_t* g = gsrc + (int64_t)((b * PB + t) * 4) * p.ldr;
        gw[b][t] = *(const uint4*)g;
        uw[b][t] = *(const uint4*)(g + F);
      }
    };
#pragma unroll
    for (int b = 0; b < DEPTH; ++b) load_batch(b);
    asm volatile("s_barrier" ::: "memory");   // every wave's fragment reads have completed (waited above)
    bf16_t* q = smem + wid * 128 * 128;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        uint2 w;
        w.x = (uint32_t)f32_to_bf16(acc[i][j][0] * p.alpha) | ((uint32_t)f32_to_bf16(acc[i][j][1] * p.alpha) << 16);
        w.y = (uint32_t)f32_to_bf16(acc[i][j][2] * p.alpha) | ((uint32_t)f32_to_bf16(acc[i][j][3] * p.alpha) << 16);
        *(uint2*)&q[(i * 16 + lr) * 128 + (((2 * j + (lk >> 1)) ^ lr) << 3) + (lk & 1) * 4] = w;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < NBATCH; ++b) {
      if (b + DEPTH < NBATCH) load_batch(b + DEPTH);
#pragma unroll
      for (int t = 0; t < PB; ++t) {
        const int r = (b * PB + t) * 4 + rsub;
        const uint4 dw = *(const uint4*)&q[r * 128 + ((c16 ^ (r & 15)) << 3)];
        const bf16_t* dv = (const bf16_t*)&dw;
        const bf16_t* gv = (const bf16_t*)&gw[b][t];
        const bf16_t* uv = (const bf16_t*)&uw[b][t];
        float dg[8], du[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          swiglu_grad(bf16_to_f32(dv[e]), bf16_to_f32(gv[e]), bf16_to_f32(uv[e]), dg[e], du[e]);
        uint4 og, ou;
        uint32_t* pg = (uint32_t*)&og;
        uint32_t* pu = (uint32_t*)&ou;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pg[e] = (uint32_t)f32_to_bf16(dg[2 * e]) | ((uint32_t)f32_to_bf16(dg[2 * e + 1]) << 16);
          pu[e] = (uint32_t)f32_to_bf16(du[2 * e]) | ((uint32_t)f32_to_bf16(du[2 * e + 1]) << 16);
        }
        bf16_t* d = dst + (int64_t)((b * PB + t) * 4) * p.ldc;
        *(uint4*)d = og;
        *(uint4*)(d + F) = ou;
      }
    }
    return;
  }
  if constexpr (EPI == 3) {
    // Softmax statistics of LM-head logits that are never stored: per row and 128-column block of
    // this wave, the max and the sum of exp(z - max) over the block's columns below N (the four
    // lanes of a row, lk = 0..3, hold 32 columns each and are merged through cross-lane shuffles),
    // and the target logit of the rows whose target lies in the block.
    const int cb = n0 + wn * 128;
    const int part = cb >> 7;
    if (p.ce_z) {
      // the logits for a backward that reads them instead of recomputing them: lane (lr, lk) holds
      // 4 consecutive columns of each (i, j) block, one 16-byte store each
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = m0 + wm * 128 + i * 16 + lr;
        if (row >= p.M) continue;
        float* zrow = p.ce_z + (int64_t)row * p.ce_ldz;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int col = cb + j * 16 + lk * 4;
          if (col + 4 <= p.N) {
            *(float4*)(zrow + col) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (col + q < p.N) zrow[col + q] = acc[i][j][q];
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm * 128 + i * 16 + lr;
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (cb + j * 16 + lk * 4 + q < p.N) mx = fmaxf(mx, acc[i][j][q]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      float se = 0.f;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (cb + j * 16 + lk * 4 + q < p.N) se += fast_expf(acc[i][j][q] - mx);
      se += __shfl_xor(se, 16);
      se += __shfl_xor(se, 32);
      if (row < p.M && cb < p.N) {
        if (lk == 0) {
          p.ce_pmax[(int64_t)row * p.ce_ldp + part] = mx;
          p.ce_psum[(int64_t)row * p.ce_ldp + part] = se;
        }
        const int64_t t = p.ce_tgt[row] - p.ce_vocab0 - cb;      // target column inside the block
        if (t >= 0 && t < 128 && cb + t < p.N && ((t >> 2) & 3) == lk) {
          float zt = 0.f;
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (j * 16 + q == (int)(t & ~12)) zt = acc[i][j][q];
          p.ce_zt[row] = zt;
        }
      }
    }
    return;
  }
  if constexpr (EPI == 4) {
    // Cross-entropy gradient of the recomputed logits: dz = bf16(w g inv_n (exp(z - lse) - onehot)),
    // the same arithmetic as the separate gradient kernel over stored logits.
    const float gs = p.ce_g[0] * p.ce_inv_n[0];
    if (m0 + BM <= p.M && n0 + BN <= p.N && (p.ldc & 7) == 0) {
      // Interior tile: each wave rounds its 128 x 128 quadrant of dz into a private 32 KB of the
      // idle LDS stages (16-byte chunk c of row r at slot c ^ (r & 15)) and stores it by rows, 16
      // lanes per 256-byte row, instead of 8 bytes per lane scattered over 16 rows.
      asm volatile("s_barrier" ::: "memory");   // every wave's fragment reads have completed
      bf16_t* qs = smem + wid * 128 * 128;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = i * 16 + lr;
        const int row = m0 + wm * 128 + r;
        const float lse = p.ce_lse[row], cf = p.ce_w[row] * gs;
        const int64_t t = p.ce_tgt[row] - p.ce_vocab0;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int col = n0 + wn * 128 + j * 16 + lk * 4;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = cf * (fast_expf(acc[i][j][e] - lse) - ((int64_t)(col + e) == t ? 1.f : 0.f));
          *(uint2*)&qs[r * 128 + (((2 * j + (lk >> 1)) ^ lr) << 3) + (lk & 1) * 4] =
              make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_wave_barrier();
      const int rsub = lane >> 4, c16 = lane & 15;
      bf16_t* dst = (bf16_t*)p.C + (int64_t)(m0 + wm * 128 + rsub) * p.ldc + n0 + wn * 128 + c16 * 8;
#pragma unroll
      for (int it = 0; it < 32; ++it) {
        const int r = it * 4 + rsub;
        *(uint4*)(dst + (int64_t)(it * 4) * p.ldc) = *(const uint4*)&qs[r * 128 + ((c16 ^ (r & 15)) << 3)];
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm * 128 + i * 16 + lr;
      if (row >= p.M) continue;
      const float lse = p.ce_lse[row], cf = p.ce_w[row] * gs;
      const int64_t t = p.ce_tgt[row] - p.ce_vocab0;
      bf16_t* crow = (bf16_t*)p.C + (int64_t)row * p.ldc;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * 128 + j * 16 + lk * 4;
        if (col >= p.N) continue;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = cf * (fast_expf(acc[i][j][q] - lse) - ((int64_t)(col + q) == t ? 1.f : 0.f));
        if (col + 4 <= p.N) {
          store4(crow + col, nullptr, v);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (col + q < p.N) crow[col + q] = f32_to_bf16(v[q]);
        }
      }
    }
    return;
  }
  if constexpr (EPI == 1) {
    // Gate/up product with 64-row interleaved weights (rows 128 b + [0, 64) = gate features
    // 64 b + [0, 64), rows 128 b + [64, 128) = the same up features): the wave's 128 columns are
    // one such pair, accumulator j < 4 the gate and j + 4 the up value of the same feature. Writes
    // C[row][64 b + c] = bf16(silu(g) u) with g, u rounded to bf16 first, as a bf16 GEMM followed
    // by the SwiGLU kernel computes it. With C2, also stores the rounded gate and up
    // values as C2[row][f] and C2[row][N/2 + f] (the [gate | up] layout of the plain product):
    // then each wave rounds its 128 x (64 gate | 64 up) block into a private 32 KB of the idle
    // LDS stages (16-byte chunks XOR-swizzled by row, as in the backward epilogue) and stores
    // both outputs by rows, 16 lanes per row: gate and up as 128-byte runs, C as one.
    // Interior tiles only (checked by the caller).
    const int f0 = (n0 + wn * 128) / 2;
    if (p.C2 == nullptr && (p.ldc & 7) == 0) {
      // Output only: each wave's 128 x 64 block goes through a private 16 KB of the idle LDS
      // stages (16-byte chunk c of row r at slot c ^ ((r >> 1) & 7)) and is stored by rows, eight
      // lanes per 128-byte row.
      asm volatile("s_barrier" ::: "memory");   // every wave's fragment reads have completed
      bf16_t* q = smem + wid * 128 * 64;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = i * 16 + lr;
#pragma unroll
        for (int j = 0; j < TN / 2; ++j) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gv = bf16_to_f32(f32_to_bf16(acc[i][j][e] * p.alpha));
            const float uv = bf16_to_f32(f32_to_bf16(acc[i][j + TN / 2][e] * p.alpha));
            v[e] = gv * sigmoidf_(gv) * uv;
          }
          *(uint2*)&q[r * 64 + (((2 * j + (lk >> 1)) ^ ((r >> 1) & 7)) << 3) + (lk & 1) * 4] =
              make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_wave_barrier();
      const int c8 = lane & 7, rs = lane >> 3;
      OutT* dst = C + (int64_t)(m0 + wm * 128 + rs) * p.ldc + f0 + 8 * c8;
#pragma unroll 4
      for (int it = 0; it < 16; ++it) {
        const int r = it * 8 + rs;
        *(uint4*)(dst + (int64_t)(it * 8) * p.ldc) = *(const uint4*)&q[r * 64 + ((c8 ^ ((r >> 1) & 7)) << 3)];
      }
      return;
    }
    if (p.C2 == nullptr) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        OutT* crow = C + (int64_t)(m0 + wm * 128 + i * 16 + lr) * p.ldc;
#pragma unroll
        for (int j = 0; j < TN / 2; ++j) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = bf16_to_f32(f32_to_bf16(acc[i][j][q] * p.alpha));
            const float uv = bf16_to_f32(f32_to_bf16(acc[i][j + TN / 2][q] * p.alpha));
            v[q] = gv * sigmoidf_(gv) * uv;
          }
          store4(crow + f0 + j * 16 + lk * 4, nullptr, v);
        }
      }
      return;
    }
    asm volatile("s_barrier" ::: "memory");   // every wave's fragment reads have completed (waited above)
    bf16_t* q = smem + wid * 128 * 128;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        uint2 w;
        w.x = (uint32_t)f32_to_bf16(acc[i][j][0] * p.alpha) | ((uint32_t)f32_to_bf16(acc[i][j][1] * p.alpha) << 16);
        w.y = (uint32_t)f32_to_bf16(acc[i][j][2] * p.alpha) | ((uint32_t)f32_to_bf16(acc[i][j][3] * p.alpha) << 16);
        *(uint2*)&q[(i * 16 + lr) * 128 + (((2 * j + (lk >> 1)) ^ lr) << 3) + (lk & 1) * 4] = w;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    const int rsub = lane >> 4, c16 = lane & 15;
    const int F = p.N / 2;
    const int64_t row0 = m0 + wm * 128 + rsub;
    bf16_t* gdst = (bf16_t*)p.C2 + row0 * p.ldc2 + (c16 < 8 ? f0 + 8 * c16 : F + f0 + 8 * (c16 - 8));
    OutT* sdst = C + row0 * p.ldc + f0 + 4 * c16;
#pragma unroll 8
    for (int it = 0; it < 32; ++it) {
      const int r = it * 4 + rsub;
      const bf16_t* qr = q + r * 128;
      const uint4 vw = *(const uint4*)&qr[(c16 ^ (r & 15)) << 3];
      const uint2 gw = *(const uint2*)&qr[(((c16 >> 1) ^ (r & 15)) << 3) + (c16 & 1) * 4];
      const uint2 uw = *(const uint2*)&qr[(((8 + (c16 >> 1)) ^ (r & 15)) << 3) + (c16 & 1) * 4];
      *(uint4*)(gdst + (int64_t)(it * 4) * p.ldc2) = vw;
      const bf16_t* gv = (const bf16_t*)&gw;
      const bf16_t* uv = (const bf16_t*)&uw;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float g = bf16_to_f32(gv[e]);
        v[e] = g * sigmoidf_(g) * bf16_to_f32(uv[e]);
      }
      store4(sdst + (int64_t)(it * 4) * p.ldc, nullptr, v);
    }
    return;
  }
  if constexpr (EPI == 5) {
    // q|k|v projection: each wave's 128 columns are one head. The quadrant is staged through LDS
    // in fp32 as for the plain epilogue; each row is then handled by 8 lanes, lane l holding
    // columns [8l, 8l+8) and their RoPE partners [64+8l, 64+8l+8): sum of squares over the head
    // (three lane shuffles), normalisation and weight, rotate_half RoPE within the lane (one
    // angle-table read serves both halves), one rounding, 16-byte stores. Interior tiles only (the
    // caller requires M and N to be multiples of 256).
    const int rsub = lane >> 3, l8 = lane & 7;
    const int64_t rowb = m0 + wm * 128 + rsub;
    const int head = (n0 + wn * 128) >> 7;
    const int nq = p.qk_nq, nqk = p.qk_nq + p.qk_nk;
    const bool isv = head >= nqk, isq = head < nq;
    const int c0 = 8 * l8;                   // first column of the lane's lower half (= angle index)
    bf16_t* dst;
    int64_t ldd;
    if (isq) { dst = (bf16_t*)p.qk_q + (int64_t)head * 128 + c0; ldd = (int64_t)nq * 128; }
    else if (!isv) { dst = (bf16_t*)p.qk_k + (int64_t)(head - nq) * 128 + c0; ldd = (int64_t)p.qk_nk * 128; }
    else { dst = (bf16_t*)p.qk_v + (int64_t)(head - nqk) * 128 + c0; ldd = (int64_t)p.qk_nk * 128; }
    bf16_t* pre = p.qk_pre && !isv ? (bf16_t*)p.qk_pre + (int64_t)head * 128 + c0 : nullptr;
    const int64_t ldp = (int64_t)nqk * 128;
    const bool norm = !isv && p.qk_wq != nullptr;
    float wv[16];
    if (norm) {
      const bf16_t* wsrc = (const bf16_t*)(isq ? p.qk_wq : p.qk_wk) + c0;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint4 u = *(const uint4*)(wsrc + 64 * hh);
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wv[8 * hh + 2 * e] = __uint_as_float(w4[e] << 16);
          wv[8 * hh + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
        }
      }
    }
    asm volatile("s_barrier" ::: "memory");   // every wave's fragment reads have completed
    float* q = (float*)smem + wid * 64 * 128;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int r = i * 16 + lr;
          f32x4_t v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[4 * h + i][j][e] * p.alpha;
          *(f32x4_t*)&q[r * 128 + (((4 * j + lk) ^ (r & 15)) << 2)] = v;
        }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_wave_barrier();
#pragma unroll 2
      for (int it = 0; it < 8; ++it) {
        const int r = it * 8 + rsub;
        float x[16];
#pragma unroll
        for (int c = 0; c < 4; ++c) {   // chunks 2 l8, 2 l8 + 1 (lower half) and 16 + 2 l8, 17 + 2 l8
          const int ch = (c < 2 ? 2 * l8 + c : 16 + 2 * l8 + (c - 2));
          const f32x4_t v = *(const f32x4_t*)&q[r * 128 + ((ch ^ (r & 15)) << 2)];
#pragma unroll
          for (int e = 0; e < 4; ++e) x[4 * c + e] = v[e];
        }
        const int64_t row = rowb + 64 * h + it * 8;
        float out[16];
        if (isv) {
#pragma unroll
          for (int e = 0; e < 16; ++e) out[e] = x[e];
        } else {
          if (pre) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
              *(uint4*)(pre + row * ldp + 64 * hh) =
                  make_uint4(pack2_bf16(x[8 * hh], x[8 * hh + 1]), pack2_bf16(x[8 * hh + 2], x[8 * hh + 3]),
                             pack2_bf16(x[8 * hh + 4], x[8 * hh + 5]), pack2_bf16(x[8 * hh + 6], x[8 * hh + 7]));
          }
          int64_t pr = p.qk_pos[row];
          pr = pr < 0 ? 0 : (pr >= p.qk_P ? p.qk_P - 1 : pr);
          const float4 ca = *(const float4*)(p.qk_cos + pr * 64 + c0), cb = *(const float4*)(p.qk_cos + pr * 64 + c0 + 4);
          const float4 sa = *(const float4*)(p.qk_sin + pr * 64 + c0), sb = *(const float4*)(p.qk_sin + pr * 64 + c0 + 4);
          const float cv[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
          const float sv[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
          if (norm) {
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) ss += x[e] * x[e];
#pragma unroll
            for (int o = 4; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            const float rs = rsqrtf(ss / 128.f + p.qk_eps);
            if (l8 == 0 && p.qk_rstd) p.qk_rstd[row * nqk + head] = rs;
#pragma unroll
            for (int e = 0; e < 16; ++e) x[e] = x[e] * rs * wv[e];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {      // rotate_half: (x, x') -> (x c - x' s, x' c + x s)
            out[e] = x[e] * cv[e] - x[8 + e] * sv[e];
            out[8 + e] = x[8 + e] * cv[e] + x[e] * sv[e];
          }
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          *(uint4*)(dst + row * ldd + 64 * hh) =
              make_uint4(pack2_bf16(out[8 * hh], out[8 * hh + 1]), pack2_bf16(out[8 * hh + 2], out[8 * hh + 3]),
                         pack2_bf16(out[8 * hh + 4], out[8 * hh + 5]), pack2_bf16(out[8 * hh + 6], out[8 * hh + 7]));
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);     // the half's reads are done before the next overwrites
      __builtin_amdgcn_wave_barrier();
    }
    return;
  }
  const bool interior = m0 + BM <= p.M && n0 + BN <= p.N && p.gate == nullptr;
  if constexpr (EPI == 0 && std::is_same<OutT, bf16_t>::value) {
    if (interior && (p.ldc & 7) == 0 && (!R || (p.ldr & 7) == 0)) {
      // Interior tile with bf16 output: each wave stages its 128 x 128 fp32 quadrant (alpha
      // applied) through a private 32 KB of the idle LDS stages, 64 rows at a time, and stores by
      // rows: 16 lanes per row, 8 columns (16 bytes) each, the residual read the same way. 16-byte
      // chunk c of staged row r sits at slot c ^ (r & 15). The residual rows of both halves are
      // loaded first, into the registers the K loop's fragments held, so their latency passes
      // once, behind the staging, instead of once per group of rows.
      const int rsub = lane >> 4, c16 = lane & 15;
      const int64_t rowb = m0 + wm * 128 + rsub;
      const int col = n0 + wn * 128 + 8 * c16;
      uint4 rw[2][16];
      if (R) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int it = 0; it < 16; ++it)
            rw[h][it] = *(const uint4*)((const bf16_t*)R + (rowb + 64 * h + it * 4) * p.ldr + col);
      }
      asm volatile("s_barrier" ::: "memory");   // every wave's fragment reads have completed
      float* q = (float*)smem + wid * 64 * 128;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int r = i * 16 + lr;
            f32x4_t v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[4 * h + i][j][e] * p.alpha;
            *(f32x4_t*)&q[r * 128 + (((4 * j + lk) ^ (r & 15)) << 2)] = v;
          }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int it = 0; it < 16; ++it) {
          const int r = it * 4 + rsub;
          const f32x4_t v0 = *(const f32x4_t*)&q[r * 128 + (((2 * c16) ^ (r & 15)) << 2)];
          const f32x4_t v1 = *(const f32x4_t*)&q[r * 128 + (((2 * c16 + 1) ^ (r & 15)) << 2)];
          const int64_t row = rowb + 64 * h + it * 4;
          float a[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          if (R) {
            const uint32_t* rp = (const uint32_t*)&rw[h][it];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              a[2 * e] += __uint_as_float(rp[e] << 16);
              a[2 * e + 1] += __uint_as_float(rp[e] & 0xffff0000u);
            }
          }
          *(uint4*)((bf16_t*)C + row * p.ldc + col) =
              make_uint4(pack2_bf16(a[0], a[1]), pack2_bf16(a[2], a[3]), pack2_bf16(a[4], a[5]), pack2_bf16(a[6], a[7]));
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);     // the half's reads are done before the next overwrites
        __builtin_amdgcn_wave_barrier();
      }
      return;
    }
  }
  if (R) {
    if (interior) epilogue(std::true_type{}, std::false_type{}); else epilogue(std::true_type{}, std::true_type{});
  } else {
    if (interior) epilogue(std::false_type{}, std::false_type{}); else epilogue(std::false_type{}, std::true_type{});
  }
}

// Row tiles per tile group (tiles are walked group by group, column by column inside a group; an
// XCD's 32 concurrent workgroups then cover group x 32/group tiles). Long-K products run faster
// with groups of 4 (measured: 16384 x 4096 x 12288 1.25 -> 1.21 ms, x 24576 2.47 -> 2.42 ms),
// the others with 8.
static int w4m16_group(int K) { return K >= 8192 ? 4 : 8; }

template <typename OutT, int EPI = 0>
static void launch_nt_w4m16(const GemmNT& p0, hipStream_t st) {
  GemmNT p = p0;
  p.group = w4m16_group(p.K + p.K2);
  constexpr size_t lds = (3 * 256 + 2 * 256) * 64 * sizeof(bf16_t);   // 160 KB
  UNOK_SET_LDS_ONCE((gemm_nt_bf16_w4m16_kernel<OutT, EPI>), lds);
  const int nb = ((p.M + 255) / 256) * ((p.N + 255) / 256);
  hipLaunchKernelGGL((gemm_nt_bf16_w4m16_kernel<OutT, EPI>), dim3(nb), dim3(256), lds, st, p);
}

// The 4-wave kernel addresses each tile's operand strips (256 rows from the tile's first) through
// buffer resources with 32-bit byte offsets and stores 4 output columns per vector (C and R rows
// aligned to 16 bytes, N a multiple of 4).
static bool buffer_ranges_ok(const GemmNT& p) {
  const int64_t lim = 0xFFFFFFFFll;
  if (p.N % 4 || p.ldc % 4 || ((uintptr_t)p.C & 15) || (p.R && (p.ldr % 4 || ((uintptr_t)p.R & 15)))) return false;
  const int64_t mr = (p.M < 256 ? p.M : 256) - 1, nr = (p.N < 256 ? p.N : 256) - 1;
  if ((mr * p.lda + p.K) * 2 > lim || (nr * p.ldb + p.K) * 2 > lim) return false;
  if (p.A2 && ((mr * p.lda2 + p.K2 + 4096) * 2 > lim || (nr * p.ldb2 + p.K2) * 2 > lim)) return false;
  return true;
}

template <int BM, int BN, int NW, int BK, int STAGES, typename OutT, bool ROT = false>
static void launch_nt_dma_t(const GemmNT& p, hipStream_t st) {
  constexpr size_t lds = (size_t)STAGES * (BM + BN) * BK * sizeof(bf16_t);
  UNOK_SET_LDS_ONCE((gemm_nt_bf16_dma_kernel<BM, BN, NW, BK, STAGES, OutT, ROT>), lds);
  const int nb = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_nt_bf16_dma_kernel<BM, BN, NW, BK, STAGES, OutT, ROT>), dim3(nb), dim3(NW * 64), lds, st, p);
}

// Large products: the 256x256 16x16x32-MFMA kernel; operands beyond its 32-bit buffer offsets
// take the 8-wave direct-to-LDS kernel, which addresses them with 64-bit pointers.
template <typename OutT>
static void launch_nt_large(const GemmNT& p, hipStream_t st) {
  if (buffer_ranges_ok(p)) launch_nt_w4m16<OutT>(p, st);
  else launch_nt_dma_t<256, 256, 8, 64, 2, OutT>(p, st);
}

// Skinny products (N <= 192): one 64 x N tile spans every output column, 4 LDS stages for
// N <= 128 and 3 for N <= 192, each workgroup's K walk rotated so that the concurrent reads
// spread over the rows' column offsets instead of all hitting the same one.
template <int BN, int STAGES>
static void launch_nt_skinny_t(const GemmNT& p, int out_dtype, hipStream_t st) {
  if (out_dtype == UNOK_F32) launch_nt_dma_t<64, BN, 4, 64, STAGES, float, true>(p, st);
  else launch_nt_dma_t<64, BN, 4, 64, STAGES, bf16_t, true>(p, st);
}

// C = alpha * gate (.) (A B^T + A2[:, seg_col] B2^T) + R.
// in_dtype: dtype of A, B, A2, B2; out_dtype: dtype of C and R.
// seg_end/seg_col: `nseg` (<= 4) extension segments over N (ignored when A2 is null).
// C[M, N/2] = silu(G) * U for the gate/up product A[M,K] B[N,K]^T with 64-row interleaved B (rows
// 128 b + [0, 64) gate, 128 b + [64, 128) up of features 64 b + [0, 64)), bf16, rounded as the
// unfused product followed by unok_swiglu_fwd. M and N multiples of 256, K of 64.
UNOK_EXPORT int unok_gemm_nt_swiglu(int M, int N, int K, const void* A, int64_t lda, const void* B, int64_t ldb,
                                    const void* A2, int64_t lda2, const void* B2, int64_t ldb2, int K2,
                                    void* C, int64_t ldc, void* gu, int64_t ldgu, void* stream) {
  UNOK_REQUIRE(M >= 0 && N >= 0 && K >= 0 && K2 >= 0, UNOK_EINVAL, "gemm_nt_swiglu: negative size M=%d N=%d K=%d",
               M, N, K);
  if (M == 0 || N == 0) return 0;
  const bool ext = A2 != nullptr && K2 > 0;
  UNOK_REQUIRE(M % 256 == 0 && N % 256 == 0 && K % 64 == 0 && K > 0 && (!ext || K2 % 32 == 0), UNOK_EINVAL,
               "gemm_nt_swiglu: M=%d and N=%d must be multiples of 256, K=%d of 64 and K2=%d of 32", M, N, K, K2);
  UNOK_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && ldc % 8 == 0 && aligned16(A) && aligned16(B) && aligned16(C) &&
                   (!ext || (lda2 % 8 == 0 && ldb2 % 8 == 0 && aligned16(A2) && aligned16(B2))) &&
                   (gu == nullptr || (ldgu % 8 == 0 && aligned16(gu))),
               UNOK_EALIGN, "gemm_nt_swiglu: row strides must be multiples of 8 and rows 16-byte aligned");
  GemmNT p{};
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb;
  p.A2 = ext ? A2 : nullptr; p.lda2 = lda2; p.B2 = B2; p.ldb2 = ldb2;
  p.C = C; p.ldc = ldc; p.C2 = gu; p.ldc2 = ldgu;
  p.M = M; p.N = N; p.K = K; p.K2 = ext ? K2 : 0; p.alpha = 1.f; p.nseg = 1;
  for (int i = 0; i < 4; ++i) { p.seg_end[i] = N; p.seg_col[i] = 0; }
  UNOK_REQUIRE(buffer_ranges_ok(p), UNOK_EINVAL, "gemm_nt_swiglu: operands exceed 32-bit buffer offsets");
  launch_nt_w4m16<bf16_t, 1>(p, (hipStream_t)stream);
  return unok::check_launch("gemm_nt_swiglu");
}

// q|k|v projection with the q/k RMSNorm and RoPE in its epilogue (bf16, head dim 128): the product
// A[M,K] B[N,K]^T (+ the LoRA extension, up to 4 segments as in unok_gemm_nt), N = 128 (nq + 2 nk),
// stays in fp32 until each q/k head is normalised (wq / wk, or neither), scaled by the weight and
// rotated; q [M, 128 nq], k and v [M, 128 nk] are written contiguous in bf16, rstd [M, nq+nk] (when
// non-null), and the q/k columns before the norm in bf16 into qk_pre [M, 128 (nq+nk)] (when
// non-null). cos_tab / sin_tab [P, 64] hold cos / sin of fl32(p * inv_freq[j]) (unok_rope_table);
// positions are clamped to [0, P). Same values as unok_gemm_nt into fp32 followed by
// unok_qknorm_rope_fwd. M and N multiples of 256, K of 64, K2 of 32.
UNOK_EXPORT int unok_gemm_nt_qkv_rope(int M, int K, int nq, int nk, const void* A, int64_t lda, const void* B,
                                      int64_t ldb, const void* A2, int64_t lda2, const void* B2, int64_t ldb2, int K2,
                                      int nseg, const int* seg_end, const int* seg_col, const void* wq, const void* wk,
                                      const int64_t* pos, const float* cos_tab, const float* sin_tab, int P, float eps,
                                      void* q_out, void* k_out, void* v_out, float* rstd, void* qk_pre, void* stream) {
  UNOK_REQUIRE(M >= 0 && K >= 0 && K2 >= 0 && nq > 0 && nk > 0 && P > 0, UNOK_EINVAL,
               "gemm_nt_qkv_rope: bad sizes M=%d K=%d nq=%d nk=%d P=%d", M, K, nq, nk, P);
  if (M == 0) return 0;
  const int N = 128 * (nq + 2 * nk);
  const bool ext = A2 != nullptr && K2 > 0;
  UNOK_REQUIRE(M % 256 == 0 && N % 256 == 0 && K % 64 == 0 && K > 0 && (!ext || K2 % 32 == 0) && nseg >= 0 &&
                   nseg <= 4 && (wq == nullptr) == (wk == nullptr),
               UNOK_EINVAL, "gemm_nt_qkv_rope: M=%d and N=%d must be multiples of 256, K=%d of 64, K2=%d of 32", M, N,
               K, K2);
  UNOK_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && aligned16(A) && aligned16(B) && aligned16(q_out) && aligned16(k_out) &&
                   aligned16(v_out) && (qk_pre == nullptr || aligned16(qk_pre)) && aligned16(cos_tab) &&
                   aligned16(sin_tab) && (!ext || (lda2 % 8 == 0 && ldb2 % 8 == 0 && aligned16(A2) && aligned16(B2))),
               UNOK_EALIGN, "gemm_nt_qkv_rope: row strides must be multiples of 8 and rows 16-byte aligned");
  GemmNT p{};
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb;
  p.A2 = ext ? A2 : nullptr; p.lda2 = lda2; p.B2 = B2; p.ldb2 = ldb2;
  p.C = q_out; p.ldc = 128 * nq;
  p.M = M; p.N = N; p.K = K; p.K2 = ext ? K2 : 0; p.alpha = 1.f;
  p.nseg = p.A2 ? (nseg > 0 ? nseg : 1) : 1;
  for (int i = 0; i < 4; ++i) { p.seg_end[i] = N; p.seg_col[i] = 0; }
  if (p.A2 && nseg > 0) {
    for (int i = 0; i < nseg; ++i) {
      p.seg_end[i] = seg_end[i]; p.seg_col[i] = seg_col[i];
      UNOK_REQUIRE(seg_col[i] % 8 == 0 && (i + 1 == nseg || seg_end[i] % 256 == 0), UNOK_EINVAL,
                   "gemm_nt_qkv_rope: segment %d (end %d, column %d) not tile-aligned", i, seg_end[i], seg_col[i]);
    }
    UNOK_REQUIRE(p.seg_end[nseg - 1] == N, UNOK_EINVAL, "gemm_nt_qkv_rope: last segment must end at N");
  }
  p.qk_q = q_out; p.qk_k = k_out; p.qk_v = v_out; p.qk_pre = qk_pre; p.qk_rstd = rstd;
  p.qk_wq = wq; p.qk_wk = wk; p.qk_pos = pos; p.qk_cos = cos_tab; p.qk_sin = sin_tab; p.qk_P = P;
  p.qk_nq = nq; p.qk_nk = nk; p.qk_eps = eps;
  UNOK_REQUIRE(buffer_ranges_ok(p), UNOK_EINVAL, "gemm_nt_qkv_rope: operands exceed 32-bit buffer offsets");
  launch_nt_w4m16<bf16_t, 5>(p, (hipStream_t)stream);
  return unok::check_launch("gemm_nt_qkv_rope");
}

// dgu[M, 2F] = SwiGLU backward of dS = A[M,K] B[F,K]^T + A2[M,K2] B2[F,K2]^T (bf16, never stored)
// against gu[M, 2F] = [gate | up]; rounded exactly as unok_gemm_nt followed by unok_swiglu_bwd.
// M and F multiples of 256, K of 64, K2 of 32.
UNOK_EXPORT int unok_gemm_nt_swiglu_bwd(int M, int F, int K, const void* A, int64_t lda, const void* B,
                                        int64_t ldb, const void* A2, int64_t lda2, const void* B2, int64_t ldb2,
                                        int K2, const void* gu, int64_t ldgu, void* dgu, int64_t lddgu,
                                        void* stream) {
  UNOK_REQUIRE(M >= 0 && F >= 0 && K >= 0 && K2 >= 0, UNOK_EINVAL, "gemm_nt_swiglu_bwd: negative size");
  if (M == 0 || F == 0) return 0;
  UNOK_REQUIRE(M % 256 == 0 && F % 256 == 0 && K % 64 == 0 && K > 0 && K2 % 32 == 0, UNOK_EINVAL,
               "gemm_nt_swiglu_bwd: M=%d and F=%d must be multiples of 256, K=%d of 64 and K2=%d of 32", M, F, K, K2);
  UNOK_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && ldgu % 8 == 0 && lddgu % 8 == 0 && aligned16(A) && aligned16(B) &&
                   aligned16(gu) && aligned16(dgu) && (K2 == 0 || (lda2 % 8 == 0 && ldb2 % 8 == 0 && aligned16(A2) &&
                                                                   aligned16(B2))),
               UNOK_EALIGN, "gemm_nt_swiglu_bwd: row strides must be multiples of 8 and rows 16-byte aligned");
  GemmNT p{};
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb;
  p.A2 = (A2 && K2 > 0) ? A2 : nullptr; p.lda2 = lda2; p.B2 = B2; p.ldb2 = ldb2;
  p.C = dgu; p.ldc = lddgu; p.R = gu; p.ldr = ldgu;
  p.M = M; p.N = F; p.K = K; p.K2 = p.A2 ? K2 : 0; p.alpha = 1.f; p.nseg = 1;
  for (int i = 0; i < 4; ++i) { p.seg_end[i] = F; p.seg_col[i] = 0; }
  UNOK_REQUIRE(buffer_ranges_ok(p), UNOK_EINVAL, "gemm_nt_swiglu_bwd: operands exceed 32-bit buffer offsets");
  launch_nt_w4m16<bf16_t, 2>(p, (hipStream_t)stream);
  return unok::check_launch("gemm_nt_swiglu_bwd");
}

// Operand checks of the LM-head loss products (H[R,K] W[V,K]^T through the 256x256 kernel, which
// addresses its operands with 32-bit buffer offsets).
static int ce_operands_ok(const char* what, int R, int V, int K, const void* H, int64_t ldh, const void* W,
                          int64_t ldw) {
  UNOK_REQUIRE(R >= 0 && V > 0 && K > 0, UNOK_EINVAL, "%s: bad size R=%d V=%d K=%d", what, R, V, K);
  UNOK_REQUIRE(K % 64 == 0 && ldh % 8 == 0 && ldw % 8 == 0 && aligned16(H) && aligned16(W), UNOK_EALIGN,
               "%s: K=%d must be a multiple of 64, row strides multiples of 8, rows 16-byte aligned", what, K);
  UNOK_REQUIRE(((int64_t)(R - 1) * ldh + K) * 2 <= 0xFFFFFFFFll && ((int64_t)(V - 1) * ldw + K) * 2 <= 0xFFFFFFFFll,
               UNOK_EINVAL, "%s: operands exceed 32-bit buffer offsets", what);
  return 0;
}

// Softmax statistics of the LM-head logits Z = H W^T (bf16 in, fp32 accumulate) without storing
// them: pmax/psum[r, b] over columns [128 b, 128 b + 128) of Z, zt[r] = Z[r, tgt[r] - vocab0] for
// targets inside [vocab0, vocab0 + V).
UNOK_EXPORT int unok_lmhead_ce_stats(int R, int V, int K, const void* H, int64_t ldh, const void* W, int64_t ldw,
                                     const int64_t* tgt, int vocab0, float* pmax, float* psum, int64_t ldp,
                                     float* zt, float* z, int64_t ldz, void* stream) {
  if (R == 0) return 0;
  int rc = ce_operands_ok("lmhead_ce_stats", R, V, K, H, ldh, W, ldw);
  if (rc) return rc;
  UNOK_REQUIRE(ldp >= (V + 127) / 128, UNOK_EINVAL, "lmhead_ce_stats: ldp=%lld < %d blocks", (long long)ldp,
               (V + 127) / 128);
  UNOK_REQUIRE(z == nullptr || (ldz >= V && ldz % 4 == 0 && aligned16(z)), UNOK_EALIGN,
               "lmhead_ce_stats: z rows must be 16-byte aligned with a stride >= V, multiple of 4 (ldz=%lld)",
               (long long)ldz);
  GemmNT p{};
  p.A = H; p.lda = ldh; p.B = W; p.ldb = ldw; p.M = R; p.N = V; p.K = K; p.alpha = 1.f; p.nseg = 1;
  for (int i = 0; i < 4; ++i) { p.seg_end[i] = V; p.seg_col[i] = 0; }
  p.ce_tgt = tgt; p.ce_vocab0 = vocab0; p.ce_pmax = pmax; p.ce_psum = psum; p.ce_ldp = ldp; p.ce_zt = zt;
  p.ce_z = z; p.ce_ldz = ldz;
  launch_nt_w4m16<float, 3>(p, (hipStream_t)stream);
  return unok::check_launch("lmhead_ce_stats");
}

// dz[r, v] = bf16(w[r] * g * inv_n * (exp(Z[r, v] - lse[r]) - [vocab0 + v == tgt[r]])) for the
// recomputed logits Z = H W^T; Z itself is never stored.
UNOK_EXPORT int unok_lmhead_ce_grad(int R, int V, int K, const void* H, int64_t ldh, const void* W, int64_t ldw,
                                    const int64_t* tgt, int vocab0, const float* lse, const float* w,
                                    const float* g, const float* inv_n, void* dz, int64_t lddz, void* stream) {
  if (R == 0) return 0;
  int rc = ce_operands_ok("lmhead_ce_grad", R, V, K, H, ldh, W, ldw);
  if (rc) return rc;
  UNOK_REQUIRE(lddz % 8 == 0 && lddz >= V && aligned16(dz), UNOK_EALIGN,
               "lmhead_ce_grad: dz rows must be 16-byte aligned with a stride >= V, multiple of 8");
  GemmNT p{};
  p.A = H; p.lda = ldh; p.B = W; p.ldb = ldw; p.C = dz; p.ldc = lddz; p.M = R; p.N = V; p.K = K; p.alpha = 1.f;
  p.nseg = 1;
  for (int i = 0; i < 4; ++i) { p.seg_end[i] = V; p.seg_col[i] = 0; }
  p.ce_tgt = tgt; p.ce_vocab0 = vocab0; p.ce_lse = lse; p.ce_w = w; p.ce_g = g; p.ce_inv_n = inv_n;
  launch_nt_w4m16<bf16_t, 4>(p, (hipStream_t)stream);
  return unok::check_launch("lmhead_ce_grad");
}

UNOK_EXPORT int unok_gemm_nt(int in_dtype, int out_dtype, int M, int N, int K,
                             const void* A, int64_t lda, const void* B, int64_t ldb,
                             const void* A2, int64_t lda2, const void* B2, int64_t ldb2, int K2,
                             int nseg, const int* seg_end, const int* seg_col,
                             void* C, int64_t ldc, const void* R, int64_t ldr,
                             const uint8_t* gate, float alpha, void* stream) {
  UNOK_REQUIRE(M >= 0 && N >= 0 && K >= 0, UNOK_EINVAL, "gemm_nt: negative size M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return 0;
  UNOK_REQUIRE(in_dtype == UNOK_F32 || in_dtype == UNOK_BF16, UNOK_EINVAL, "gemm_nt: bad in_dtype %d", in_dtype);
  UNOK_REQUIRE(out_dtype == UNOK_F32 || out_dtype == UNOK_BF16, UNOK_EINVAL, "gemm_nt: bad out_dtype %d", out_dtype);
  UNOK_REQUIRE(nseg >= 0 && nseg <= 4, UNOK_EINVAL, "gemm_nt: nseg=%d outside [0,4]", nseg);
  GemmNT p{};
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb;
  p.A2 = (A2 && K2 > 0) ? A2 : nullptr; p.lda2 = lda2; p.B2 = B2; p.ldb2 = ldb2;
  p.C = C; p.ldc = ldc; p.R = R; p.ldr = ldr; p.gate = gate;
  p.M = M; p.N = N; p.K = K; p.K2 = p.A2 ? K2 : 0; p.alpha = alpha;
  p.nseg = p.A2 ? (nseg > 0 ? nseg : 1) : 1;
  for (int i = 0; i < 4; ++i) { p.seg_end[i] = N; p.seg_col[i] = 0; }
  if (p.A2 && nseg > 0) {
    for (int i = 0; i < nseg; ++i) { p.seg_end[i] = seg_end[i]; p.seg_col[i] = seg_col[i]; }
    UNOK_REQUIRE(p.seg_end[nseg - 1] == N, UNOK_EINVAL, "gemm_nt: last segment must end at N");
  }
  hipStream_t st = (hipStream_t)stream;
  if (in_dtype == UNOK_F32) {
    // The fp32 kernel uses 64-wide N tiles; segment boundaries must align to them.
    for (int i = 0; p.A2 && i + 1 < p.nseg; ++i)
      UNOK_REQUIRE(p.seg_end[i] % 64 == 0, UNOK_EINVAL, "gemm_nt(f32): segment end %d not a multiple of 64", p.seg_end[i]);
    dim3 grid((N + 63) / 64, (M + 63) / 64);
    if (out_dtype == UNOK_BF16)
      hipLaunchKernelGGL((gemm_nt_f32_kernel<bf16_t>), grid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((gemm_nt_f32_kernel<float>), grid, dim3(256), 0, st, p);
    return unok::check_launch("gemm_nt_f32");
  }
  // bf16 MFMA path: 16-byte vector loads need K-contiguous rows with 8-element granularity.
  UNOK_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && aligned16(A) && aligned16(B), UNOK_EALIGN,
               "gemm_nt(bf16): K=%d lda=%lld ldb=%lld must be multiples of 8 and A/B 16-byte aligned", K,
               (long long)lda, (long long)ldb);
  if (p.A2) {
    UNOK_REQUIRE(K2 % 8 == 0 && lda2 % 8 == 0 && ldb2 % 8 == 0 && aligned16(A2) && aligned16(B2), UNOK_EALIGN,
                 "gemm_nt(bf16): extension K2=%d lda2=%lld ldb2=%lld must be multiples of 8", K2,
                 (long long)lda2, (long long)ldb2);
    for (int i = 0; i < p.nseg; ++i)
      UNOK_REQUIRE(p.seg_col[i] % 8 == 0, UNOK_EALIGN, "gemm_nt(bf16): segment column %d not a multiple of 8", p.seg_col[i]);
  }
  // Tile choice: the largest tile whose N-segment boundaries stay tile-aligned.
  auto segs_ok = [&](int bn) {
    for (int i = 0; p.A2 && i + 1 < p.nseg; ++i) if (p.seg_end[i] % bn) return false;
    return true;
  };
  const long long big_tiles = (long long)((M + 255) / 256) * ((N + 255) / 256);
  if (N <= 192 && !p.A2 && K % 64 == 0 && M >= 4096) {
    // Skinny products (LoRA x·Aᵀ and dY·B, N = r .. 3r): every activation row is read from HBM once.
    // (N = 256 and 384 run faster on the 128x128 and 256x256 kernels: 116 / 105 us against 135 /
    // 208 us for a 64 x N tile at 32768 x 4096.)
    const int bn = (N + 63) / 64 * 64;
    if (bn == 64) launch_nt_skinny_t<64, 4>(p, out_dtype, st);
    else if (bn == 128 && M >= 32768 && K >= 8192) {
      // many rows and a long K (the rank-128 products over the 12288-wide FFN side at 8 x 4096
      // rows): 128-row tiles of 8 waves read each weight tile from L2 half as often (221 against
      // 260 us at 32768 x 128 x 12288; at 4096-deep or 16384-row shapes they do not pay)
      if (out_dtype == UNOK_F32) launch_nt_dma_t<128, 128, 8, 64, 3, float, true>(p, st);
      else launch_nt_dma_t<128, 128, 8, 64, 3, bf16_t, true>(p, st);
    } else if (bn == 128) launch_nt_skinny_t<128, 4>(p, out_dtype, st);
    else launch_nt_skinny_t<192, 3>(p, out_dtype, st);
  } else if (N <= 64 || !segs_ok(128)) {
    UNOK_REQUIRE(segs_ok(64), UNOK_EINVAL, "gemm_nt(bf16): segment ends must be multiples of 64");
    launch_nt_bf16<128, 64>(p, out_dtype, st);
  } else if (N <= 128 || !segs_ok(256) || big_tiles < (K >= 8192 ? 192 : 256)) {
    // (a long-K product keeps the 256x256 kernel down to three quarters of a tile per CU)
    if ((long long)((M + 127) / 128) * ((N + 127) / 128) < 256) launch_nt_bf16<64, 128>(p, out_dtype, st);
    else launch_nt_bf16<128, 128>(p, out_dtype, st);
  } else if (K % 64 == 0 && (!p.A2 || p.K2 % 32 == 0)) {
    if (out_dtype == UNOK_F32) launch_nt_large<float>(p, st); else launch_nt_large<bf16_t>(p, st);
  } else {
    launch_nt_bf16<256, 256>(p, out_dtype, st);
  }
  return unok::check_launch("gemm_nt_bf16");
}

// Workspace bytes gemm_tn needs for a given problem (partials of the split-K reduction).
// Split counts of the two TN kernels; the workspace is sized for the larger one.
static int tn_general_splits(int Mrows, int P, int Q) {
  const int64_t tiles = (int64_t)((P + 63) / 64) * ((Q + 63) / 64);
  int64_t nsplit = (512 + tiles - 1) / tiles;
  const int64_t max_split = (Mrows + 255) / 256;
  if (nsplit > max_split) nsplit = max_split;
  return nsplit < 1 ? 1 : (int)nsplit;
}

// Skinny TN product with both operands read as columns of row-major LDS tiles: per workgroup,
// out tile [NS x 128] (rows s of the skinny operand S, columns x0 .. x0 + 127 of the wide operand
// X) over one split of the token rows. 64-row tiles of X (128 columns) and S (NS columns) stream
// into two LDS stages by direct-to-LDS loads (kswz-swizzled rows); every MFMA operand is an LDS
// transpose load of 16 rows (the same permuted row order for both operands, so the products
// pair up). Wave w owns x columns x0 + 32 w .. + 31 and all NS / 32 row blocks. Partials are
// written as WS[z][s][x] (TOUT: WS[z][x][s]), for the split-K reduction. Four
// workgroups per CU for NS = 32 (40 KB of LDS each) and three for NS = 64 (48 KB), so the split
// counts of the LoRA shapes (e.g. 96 strips x 6 splits for 12288 columns) run in one round; two
// for NS = 96 .. 192 (56 .. 80 KB).
template <int NS, bool TOUT>
__global__ __launch_bounds__(256, NS == 32 ? 4 : NS == 64 ? 3 : 2) void gemm_tn_tr_kernel(const GemmTNSkinny p) {
  constexpr int BK = 64, XB = 128, TS = NS / 32;
  // The skinny operand's tile is one swizzled [64 x NSA] tile (NSA = 128, 64 or 32) and, for
  // NS = 96, 160 and 192, a second [64 x NSB] one (NSB = 32 or 64) holding the columns past NSA.
  constexpr int NSA = NS >= 128 ? 128 : NS >= 64 ? 64 : 32, NSB = NS - NSA, TSA = NSA / 32;
  constexpr int NSB_ = NSB > 0 ? NSB : 64;   // tile width for the helpers (unused when NSB = 0)
  static_assert(NS == 32 || NS == 64 || NS == 96 || NS == 128 || NS == 160 || NS == 192,
                "skinny side of 32, 64, 96 (64 + 32), 128, 160 (128 + 32) or 192 (128 + 64) columns");
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];
  bf16_t* Xs = smem;                   // [2][BK * XB]
  bf16_t* Ss = smem + 2 * BK * XB;     // [2][BK * NSA]
  bf16_t* Sb = Ss + 2 * BK * NSA;      // [2][BK * NSB]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, lq = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(w);
  const int nstrip = (p.NX + XB - 1) / XB;
  const int lin = xcd_remap(blockIdx.x, gridDim.x);
  const int x0 = (lin % nstrip) * XB, z = lin / nstrip;
  const int mbeg = z * p.rows_per_split;
  const int mend = min(p.Mrows, mbeg + p.rows_per_split);
  const int nt = mend > mbeg ? (mend - mbeg + BK - 1) / BK : 0;
  const uint32_t xo = dma_lane_off<XB>(p.ldx, x0, wid, lane), so = dma_lane_off<NSA>(p.lds, 0, wid, lane);
  const uint32_t sob = NSB > 0 ? dma_lane_off<NSB_>(p.lds, NSA, wid, lane) : 0u;
  auto fetch = [&](int t) {
    const int m0 = mbeg + t * BK;
    dma_tile<XB>(p.X, p.ldx, xo, m0, mend, Xs + (t & 1) * BK * XB, wid);
    dma_tile<NSA>(p.S, p.lds, so, m0, mend, Ss + (t & 1) * BK * NSA, wid);
    if constexpr (NSB > 0) dma_tile<NSB_>(p.S, p.lds, sob, m0, mend, Sb + (t & 1) * BK * NSB_, wid);
  };
  const int2 xoff = tr_frag_off<XB>(w, lane);
  int2 soff[TS];
#pragma unroll
  for (int i = 0; i < TS; ++i) soff[i] = i < TSA ? tr_frag_off<NSA>(i, lane) : tr_frag_off<NSB_>(i - TSA, lane);
  f32x16_t acc[TS];
#pragma unroll
  for (int i = 0; i < TS; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  if (nt > 0) fetch(0);
#pragma unroll 1
  for (int t = 0; t < nt; ++t) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();                       // tile t in LDS; every wave is done with tile t-1
    if (t + 1 < nt) fetch(t + 1);
    const uint32_t xb = lds_addr(Xs + (t & 1) * BK * XB), sb = lds_addr(Ss + (t & 1) * BK * NSA);
    const uint32_t sbb = lds_addr(Sb + (t & 1) * BK * NSB_);
    // All operands of the tile's four 16-row steps, then one wait, then the MFMAs.
    u32x2_t xl[4], xh[4], sl[4][TS], sh[4][TS];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      tr_issue_p<XB>(make_uint2(xb + 2 * xoff.x, xb + 2 * xoff.y), q, xl[q], xh[q]);
#pragma unroll
      for (int i = 0; i < TS; ++i) {
        if (i < TSA) tr_issue_p<NSA>(make_uint2(sb + 2 * soff[i].x, sb + 2 * soff[i].y), q, sl[q][i], sh[q][i]);
        else tr_issue_p<NSB_>(make_uint2(sbb + 2 * soff[i].x, sbb + 2 * soff[i].y), q, sl[q][i], sh[q][i]);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // The results pass through these empty statements after the wait, so nothing reads them earlier.
      asm volatile("" : "+v"(xl[q]), "+v"(xh[q]));
      const bf16x8_t xf = tr_join(xl[q], xh[q]);
#pragma unroll
      for (int i = 0; i < TS; ++i) {
        asm volatile("" : "+v"(sl[q][i]), "+v"(sh[q][i]));
        const bf16x8_t sf = tr_join(sl[q][i], sh[q][i]);
        acc[i] = TOUT ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf, sf, acc[i], 0, 0, 0)
                      : __builtin_amdgcn_mfma_f32_32x32x16_bf16(sf, xf, acc[i], 0, 0, 0);
      }
    }
  }

  if (TOUT) {
    // acc[i][r] = result[x = x0 + 32 w + 8 (r / 4) + 4 g + r % 4][s = 32 i + lq]
    float* W = p.WS + (int64_t)z * p.NX * NS;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int x = x0 + w * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
      if (x < p.NX) {
#pragma unroll
        for (int i = 0; i < TS; ++i) W[(int64_t)x * NS + i * 32 + lq] = acc[i][r] * p.alpha;
      }
    }
  } else {
    // acc[i][r] = result[s = 32 i + 8 (r / 4) + 4 g + r % 4][x = x0 + 32 w + lq]
    const int col = x0 + w * 32 + lq;
    if (col < p.NX) {
      float* W = p.WS + (int64_t)z * NS * p.NX + col;
#pragma unroll
      for (int i = 0; i < TS; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = i * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
          W[(int64_t)row * p.NX] = acc[i][r] * p.alpha;
        }
    }
  }
}

template <int NS>
static void launch_tn_tr_t(const GemmTNSkinny& p, int nz, bool tout, hipStream_t st) {
  constexpr size_t lds = 2 * 64 * (128 + NS) * sizeof(bf16_t);
  UNOK_SET_LDS_ONCE((gemm_tn_tr_kernel<NS, true>), lds);
  UNOK_SET_LDS_ONCE((gemm_tn_tr_kernel<NS, false>), lds);
  const int nstrip = (p.NX + 127) / 128;
  if (tout)
    hipLaunchKernelGGL((gemm_tn_tr_kernel<NS, true>), dim3(nstrip * nz), dim3(256), lds, st, p);
  else
    hipLaunchKernelGGL((gemm_tn_tr_kernel<NS, false>), dim3(nstrip * nz), dim3(256), lds, st, p);
}

// Wide rank side (NS = 256 or 384: the 2r / 3r LoRA groups at rank 128): the tiles, row splits and
// partial layout of gemm_tn_tr_kernel, with the waves split over S instead of X. Wave w owns the
// S columns [NS/4 w, NS/4 (w + 1)) (NS/128 blocks of 32) against all 128 X columns of the strip,
// so a 16-row step reads 4 + NS/128 transpose-loaded fragments for 4 NS/128 MFMAs (the X-split
// layout would read 1 + NS/32 for NS/32 and run into the LDS read bandwidth). The S tile is kept
// as NS/128 swizzled [64 x 128] tiles; two stages take 96 KB (NS = 256) or 128 KB (NS = 384) of
// LDS, one workgroup per CU.
template <int NS, bool TOUT>
__global__ __launch_bounds__(256, 1) void gemm_tn_trw_kernel(const GemmTNSkinny p) {
  constexpr int BK = 64, XB = 128, NT = NS / 128, TSW = NS / 128;
  static_assert(NS == 256 || NS == 384, "wide skinny side of 256 or 384 columns");
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];
  bf16_t* Xs = smem;                   // [2][BK * XB]
  bf16_t* Ss = smem + 2 * BK * XB;     // [2][NT][BK * 128]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, lq = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(w);
  const int nstrip = (p.NX + XB - 1) / XB;
  const int lin = xcd_remap(blockIdx.x, gridDim.x);
  const int x0 = (lin % nstrip) * XB, z = lin / nstrip;
  const int mbeg = z * p.rows_per_split;
  const int mend = min(p.Mrows, mbeg + p.rows_per_split);
  const int nt = mend > mbeg ? (mend - mbeg + BK - 1) / BK : 0;
  const uint32_t xo = dma_lane_off<XB>(p.ldx, x0, wid, lane);
  uint32_t so[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) so[j] = dma_lane_off<128>(p.lds, 128 * j, wid, lane);
  auto fetch = [&](int t) {
    const int m0 = mbeg + t * BK;
    dma_tile<XB>(p.X, p.ldx, xo, m0, mend, Xs + (t & 1) * BK * XB, wid);
#pragma unroll
    for (int j = 0; j < NT; ++j) dma_tile<128>(p.S, p.lds, so[j], m0, mend, Ss + ((t & 1) * NT + j) * BK * 128, wid);
  };
  int2 xoff[4], soff[TSW];
#pragma unroll
  for (int i = 0; i < 4; ++i) xoff[i] = tr_frag_off<XB>(i, lane);
#pragma unroll
  for (int j = 0; j < TSW; ++j) {
    const int sb = TSW * wid + j;              // this wave's S block j: tile sb / 4, block sb % 4 within it
    const int2 o = tr_frag_off<128>(sb & 3, lane);
    soff[j] = make_int2(o.x + (sb >> 2) * BK * 128, o.y + (sb >> 2) * BK * 128);
  }
  f32x16_t acc[4][TSW];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < TSW; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (nt > 0) fetch(0);
#pragma unroll 1
  for (int t = 0; t < nt; ++t) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();                       // tile t in LDS; every wave is done with tile t-1
    if (t + 1 < nt) fetch(t + 1);
    const uint32_t xb = lds_addr(Xs + (t & 1) * BK * XB), sb = lds_addr(Ss + (t & 1) * NT * BK * 128);
    u32x2_t xl[4][4], xh[4][4], sl[4][TSW], sh[4][TSW];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        tr_issue_p<XB>(make_uint2(xb + 2 * xoff[i].x, xb + 2 * xoff[i].y), q, xl[q][i], xh[q][i]);
#pragma unroll
      for (int j = 0; j < TSW; ++j)
        tr_issue_p<128>(make_uint2(sb + 2 * soff[j].x, sb + 2 * soff[j].y), q, sl[q][j], sh[q][j]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // The results pass through these empty statements after the wait, so nothing reads them earlier.
      bf16x8_t xf[4], sf[TSW];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        asm volatile("" : "+v"(xl[q][i]), "+v"(xh[q][i]));
        xf[i] = tr_join(xl[q][i], xh[q][i]);
      }
#pragma unroll
      for (int j = 0; j < TSW; ++j) {
        asm volatile("" : "+v"(sl[q][j]), "+v"(sh[q][j]));
        sf[j] = tr_join(sl[q][j], sh[q][j]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TSW; ++j)
          acc[i][j] = TOUT ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[i], sf[j], acc[i][j], 0, 0, 0)
                           : __builtin_amdgcn_mfma_f32_32x32x16_bf16(sf[j], xf[i], acc[i][j], 0, 0, 0);
    }
  }

  if (TOUT) {
    // acc[i][j][r] = result[x = x0 + 32 i + 8 (r / 4) + 4 g + r % 4][s = 32 (TSW w + j) + lq]
    float* W = p.WS + (int64_t)z * p.NX * NS;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int x = x0 + i * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
        if (x < p.NX) {
#pragma unroll
          for (int j = 0; j < TSW; ++j) W[(int64_t)x * NS + (TSW * w + j) * 32 + lq] = acc[i][j][r] * p.alpha;
        }
      }
  } else {
    // acc[i][j][r] = result[s = 32 (TSW w + j) + 8 (r / 4) + 4 g + r % 4][x = x0 + 32 i + lq]
    float* W = p.WS + (int64_t)z * NS * p.NX;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = x0 + i * 32 + lq;
      if (col < p.NX) {
#pragma unroll
        for (int j = 0; j < TSW; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = (TSW * w + j) * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
            W[(int64_t)row * p.NX + col] = acc[i][j][r] * p.alpha;
          }
      }
    }
  }
}

template <int NS>
static void launch_tn_trw_t(const GemmTNSkinny& p, int nz, bool tout, hipStream_t st) {
  constexpr size_t lds = 2 * 64 * (128 + NS) * sizeof(bf16_t);
  UNOK_SET_LDS_ONCE((gemm_tn_trw_kernel<NS, true>), lds);
  UNOK_SET_LDS_ONCE((gemm_tn_trw_kernel<NS, false>), lds);
  const int nstrip = (p.NX + 127) / 128;
  if (tout)
    hipLaunchKernelGGL((gemm_tn_trw_kernel<NS, true>), dim3(nstrip * nz), dim3(256), lds, st, p);
  else
    hipLaunchKernelGGL((gemm_tn_trw_kernel<NS, false>), dim3(nstrip * nz), dim3(256), lds, st, p);
}

// Row splits of the transpose-load TN kernels: about one round of workgroups (4 per CU for NS = 32,
// 3 for NS = 64, 2 for NS = 96 .. 192, 1 for NS = 256 and 384 on 256 CUs), at most 16 splits for wide sides
// (2048 columns and more, where the partials and their reduction would grow faster than the
// parallelism helps) and 64 otherwise, at least 256 rows per split.
static int tn_tr_splits(int Mrows, int NX, int NS) {
  const int nstrip = (NX + 127) / 128;
  const int slots = NS == 32 ? 1024 : NS == 64 ? 768 : NS <= 192 ? 512 : 256;
  int nz = slots / nstrip;
  const int cap = NX >= 2048 ? 16 : 64;
  if (nz > cap) nz = cap;
  const int max_split = (Mrows + 255) / 256;
  if (nz > max_split) nz = max_split;
  return nz < 1 ? 1 : nz;
}

UNOK_EXPORT int64_t unok_gemm_tn_workspace(int Mrows, int P, int Q) {
  const int a = tn_general_splits(Mrows, P, Q);
  const int c = tn_tr_splits(Mrows, P <= Q ? Q : P, P <= Q ? P : Q);
  return (int64_t)(a > c ? a : c) * P * Q * 4;
}

// Rank-side widths of the skinny path: 32 .. 192 in steps of 32 on the transpose-load kernel,
// 256 and 384 on its wide variant; other widths take the general TN kernel.
static bool tn_skinny_width(int NS) { return (NS % 32 == 0 && NS <= 192) || NS == 256 || NS == 384; }

static void launch_tn_skinny(const GemmTNSkinny& p, int nz, bool tout, hipStream_t st) {
  switch (p.NS) {
    case 32: launch_tn_tr_t<32>(p, nz, tout, st); break;
    case 64: launch_tn_tr_t<64>(p, nz, tout, st); break;
    case 96: launch_tn_tr_t<96>(p, nz, tout, st); break;
    case 128: launch_tn_tr_t<128>(p, nz, tout, st); break;
    case 160: launch_tn_tr_t<160>(p, nz, tout, st); break;
    case 192: launch_tn_tr_t<192>(p, nz, tout, st); break;
    case 256: launch_tn_trw_t<256>(p, nz, tout, st); break;
    default: launch_tn_trw_t<384>(p, nz, tout, st); break;
  }
}

// C[P,Q] (fp32, row stride ldc) = beta * C + alpha * A[Mrows,P]^T B[Mrows,Q]
UNOK_EXPORT int unok_gemm_tn(int in_dtype, int Mrows, int P, int Q, const void* A, int64_t lda,
                             const void* B, int64_t ldb, float* C, int64_t ldc, float alpha, float beta,
                             void* workspace, int64_t ws_bytes, void* stream) {
  UNOK_REQUIRE(Mrows >= 0 && P >= 0 && Q >= 0, UNOK_EINVAL, "gemm_tn: negative size");
  if (P == 0 || Q == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  const int64_t need = unok_gemm_tn_workspace(Mrows, P, Q);
  UNOK_REQUIRE(workspace != nullptr && ws_bytes >= need, UNOK_EINVAL,
               "gemm_tn: workspace of %lld bytes needed, %lld given", (long long)need, (long long)ws_bytes);
  if (in_dtype == UNOK_BF16 && Mrows > 0) {
    // Skinny path: the rank side (tn_skinny_width) against a wide operand.
    const bool a_small = P <= Q;
    const int NS = a_small ? P : Q, NX = a_small ? Q : P;
    const int64_t lds_ = a_small ? lda : ldb, ldx = a_small ? ldb : lda;
    const void* S = a_small ? A : B;
    const void* X = a_small ? B : A;
    if (tn_skinny_width(NS) && NX >= TNS_MIN_NX && NX % 8 == 0 && lds_ % 8 == 0 && ldx % 8 == 0 && aligned16(S) &&
        aligned16(X)) {
      const int nz0 = tn_tr_splits(Mrows, NX, NS);
      int rps = (Mrows + nz0 - 1) / nz0;
      rps = ((rps + TNS_BK - 1) / TNS_BK) * TNS_BK;
      const int nz = (Mrows + rps - 1) / rps;
      GemmTNSkinny q{(const bf16_t*)S, lds_, (const bf16_t*)X, ldx, (float*)workspace, Mrows, NS, NX, rps, alpha};
      launch_tn_skinny(q, nz, !a_small, st);
      int rc = unok::check_launch("gemm_tn_skinny");
      if (rc) return rc;
      const int blocks = reduce_blocks(P, Q);
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, (const float*)workspace, C, ldc,
                         P, Q, nz, beta);
      return unok::check_launch("gemm_tn_reduce");
    }
  }
  const int nsplit = tn_general_splits(Mrows, P, Q);
  int rps = (Mrows + nsplit - 1) / nsplit;
  rps = ((rps + 63) / 64) * 64;
  if (rps == 0) rps = 64;
  const int nz = Mrows > 0 ? (Mrows + rps - 1) / rps : 1;
  GemmTN p{A, lda, B, ldb, (float*)workspace, Mrows, P, Q, rps, alpha};
  if (in_dtype == UNOK_F32) {
    dim3 grid(((P + 63) / 64) * ((Q + 63) / 64), nz);
    hipLaunchKernelGGL(gemm_tn_f32_kernel, grid, dim3(256), 0, st, p);
  } else {
    UNOK_REQUIRE(in_dtype == UNOK_BF16, UNOK_EINVAL, "gemm_tn: bad dtype %d", in_dtype);
    UNOK_REQUIRE(P % 8 == 0 && Q % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && aligned16(A) && aligned16(B),
                 UNOK_EALIGN, "gemm_tn(bf16): P, Q, lda, ldb must be multiples of 8 (P=%d Q=%d)", P, Q);
    if (P <= Q) {
      dim3 grid(((P + 63) / 64) * ((Q + 255) / 256), nz);
      hipLaunchKernelGGL((gemm_tn_bf16_kernel<64, 256>), grid, dim3(256), 0, st, p);
    } else {
      dim3 grid(((P + 255) / 256) * ((Q + 63) / 64), nz);
      hipLaunchKernelGGL((gemm_tn_bf16_kernel<256, 64>), grid, dim3(256), 0, st, p);
    }
  }
  int rc = unok::check_launch("gemm_tn");
  if (rc) return rc;
  const int blocks = reduce_blocks(P, Q);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, (const float*)workspace, C, ldc, P, Q, nz, beta);
  return unok::check_launch("gemm_tn_reduce");
}

// ---------------------------------------------------------------------------------------
// unok_gemm_tn_noalloc: unok_gemm_tn with its split-K partials in a library-held device array
// instead of a caller workspace, for callers that cannot allocate device memory. The array is a
// file-scope __device__ object, so every GPU the library runs on holds its own copy (64 MiB)
// until the process ends. Its device address is resolved once per device, with that device
// current, by hipGetSymbolAddress on the first call there; the host-side name `scratch` is never
// passed to a kernel. Every split writes all of its partials before the reduction reads them, so
// nothing has to be cleared between calls; calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------------------
#include <mutex>

#define UNOK_TN_SCRATCH_BYTES ((int64_t)64 << 20)
static __device__ __align__(256) float scratch[UNOK_TN_SCRATCH_BYTES / 4];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices];   // device address of `scratch`, per device (null: not yet resolved)
}  // namespace

static int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return unok::set_error((int)e, "gemm_tn_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  UNOK_REQUIRE(dev >= 0 && dev < kScratchDevices, UNOK_EUNSUPPORTED, "gemm_tn_noalloc: device %d beyond the %d supported",
               dev, kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return unok::set_error(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol,
                             "gemm_tn_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                             hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

UNOK_EXPORT int unok_gemm_tn_noalloc(int in_dtype, int Mrows, int P, int Q, const void* A, int64_t lda,
                                     const void* B, int64_t ldb, float* C, int64_t ldc, float alpha, float beta,
                                     void* stream) {
  UNOK_REQUIRE(Mrows >= 0 && P >= 0 && Q >= 0, UNOK_EINVAL, "gemm_tn_noalloc: negative size");
  if (P == 0 || Q == 0) return 0;
  const int64_t need = unok_gemm_tn_workspace(Mrows, P, Q);
  UNOK_REQUIRE(need <= UNOK_TN_SCRATCH_BYTES, UNOK_EINVAL,
               "gemm_tn_noalloc: Mrows=%d P=%d Q=%d needs %lld bytes of split-K scratch; the library holds %lld",
               Mrows, P, Q, (long long)need, (long long)UNOK_TN_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  return unok_gemm_tn(in_dtype, Mrows, P, Q, A, lda, B, ldb, C, ldc, alpha, beta, ws, UNOK_TN_SCRATCH_BYTES, stream);
}
