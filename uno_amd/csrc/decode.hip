// Few-row products of decode and draft blocks.
//
// A draft block of the two-pass decoder runs every linear layer on B x L rows (128 for 8 sequences
// of 16 rows): the product is a stream of the weight matrix past a small activation tile. The
// training GEMMs tile M and N and give each workgroup the whole K walk; at 128 rows that leaves
// a few dozen workgroups for a 4096-wide output and most of the chip idle. Here every workgroup
// owns one 128 x 128 output tile and a contiguous range of the K tiles, so the grid is
// (output tiles) x (K ranges) and fills all CUs while each weight element is still read once.
//
// The gated LoRA update y += (m (.) x A^T) (s B)^T rides along: the rows of A are extra output
// columns of the same product (they share the activation stream), and the kernel that adds the K
// ranges' fp32 partial sums (in range order, so the result does not depend on which workgroup
// finished first) also forms the hidden h = bf16(m (.) x A^T) of its rows and applies the rank-r
// update and the epilogue. With one K range and no LoRA the product kernel writes C itself.
#include "common.h"

namespace {

// Output tile 128 x 128, K tile 128; the weight streams through RB_D + 1 register sets (RB_D tiles
// in flight), the activation tiles through RB_D + 1 LDS stages.
constexpr int RB_M = 128, RB_N = 128, RB_K = 128, RB_W = 4, RB_D = 3;

struct RowsGemm {
  const bf16_t* A; int64_t lda;      // [M, K] activations
  const bf16_t* B; int64_t ldb;      // [N, K] weight
  const bf16_t* LA; int64_t ldla;    // [R, K] LoRA A rows: output columns N .. N + R of the product
  int M, N, K, R;
  int splits;                        // K ranges
  float* ws; int64_t ldw;            // [splits][M][ldw = N + R] fp32 partial sums (split path)
  bf16_t* C; int64_t ldc;            // direct path output
  const bf16_t* Res; int64_t ldres;  // direct path residual
};

// 16 bytes from global memory straight into LDS: lane l writes lds_wave_base + 16 l.
__device__ __forceinline__ void dma16(const void* g, bf16_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N) through the builtin (expcnt and lgkmcnt left at their maxima), so that the
// compiler's own wait placement knows the loads it covers have completed.
template <int N> __device__ __forceinline__ void rows_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Grid: one workgroup per (K range, output column tile, output row tile), row tiles fastest so
// that the row tiles of one weight tile run on the same XCD. Column tiles past N cover the LoRA A
// rows. Wave w owns output columns 32 w + [0, 32) of the tile for all 128 rows: four 32x32x16 MFMA
// accumulators, whose second operand (32 weight rows x 16 k) it loads straight from global memory
// into registers, RB_D K tiles ahead (8 x 16 bytes per lane and tile); the 128 x 128 activation
// tile, which all four waves read, goes to LDS by direct-to-LDS loads. A lane's eight weight
// loads cover 128 contiguous bytes of its row (lane groups 0 / 1 take k 0-63 / 64-127), so MFMA
// step j multiplies k = 64 g + 8 j + [0, 8) of lane group g; the activation fragments use the same
// order. Rows beyond M and columns beyond N (R) are clamped to the last valid row and never
// stored. The activation row r's 16-byte chunk c sits in LDS slot c ^ (r % 16).
template <bool DIRECT>
__global__ __launch_bounds__(RB_W * 64) void gemm_nt_rows_kernel(const RowsGemm p) {
  constexpr int BM = RB_M, BN = RB_N, BK = RB_K, D = RB_D, AS = RB_D + 1;
  constexpr int ACH = BK / 8;                       // 16-byte chunks per activation row
  constexpr int A_INS = BM * ACH / (RB_W * 64);     // direct-to-LDS loads per wave and tile (4 rows each)
  constexpr int W_INS = 8;                          // weight loads per lane and tile
  constexpr int LPT = A_INS + W_INS;
  static_assert(A_INS == 8 && (D - 1) * LPT < 64, "tile shape");
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];

  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nM = (p.M + BM - 1) / BM, nNm = (p.N + BN - 1) / BN;
  const int nN = nNm + (p.LA ? (p.R + BN - 1) / BN : 0);
  const int lin = xcd_remap(blockIdx.x, nM * nN * p.splits);
  const int tm = lin % nM, tn = (lin / nM) % nN, split = lin / (nM * nN);
  const int m0 = tm * BM;
  const bool lora_tile = tn >= nNm;
  // this tile's columns: weight rows n0 .. of B, or LoRA A rows n0 .. of LA (output columns N + n0 ..)
  const int n0 = (lora_tile ? tn - nNm : tn) * BN;
  const int ncols = lora_tile ? p.R : p.N;

  const int nk = p.K / BK;
  const int kb = (int)((int64_t)split * nk / p.splits), ke = (int)((int64_t)(split + 1) * nk / p.splits);

  const int arow_in = lane >> 4, aslot = lane & 15;   // direct-to-LDS lane: tile row 4 (4 i + w) + lane / 16
  const int lg = lane >> 5;
  const int wn = min(n0 + wid * 32 + (lane & 31), ncols - 1);
  const bf16_t* wrow = (lora_tile ? p.LA + (int64_t)wn * p.ldla : p.B + (int64_t)wn * p.ldb) + lg * 64;

  auto issue_a = [&](int t, int stage) {
    bf16_t* as = smem + stage * BM * BK;
    const int kk = t * BK;
#pragma unroll
    for (int i = 0; i < A_INS; ++i) {
      const int r = (i * RB_W + wid) * 4 + arow_in;
      const int gm = min(m0 + r, p.M - 1);
      dma16(p.A + (int64_t)gm * p.lda + kk + ((aslot ^ (r & 15)) << 3), as + (i * RB_W + wid) * 4 * BK);
    }
  };
  auto issue_w = [&](int t, bf16x8_t (&w)[W_INS]) {
    const int kk = t * BK;
#pragma unroll
    for (int j = 0; j < W_INS; ++j) w[j] = *(const bf16x8_t*)(wrow + kk + j * 8);
  };

  f32x16_t acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  auto mfma_step = [&](const bf16_t* as, int chunk, const bf16x8_t& w) {
    bf16x8_t a[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int r = mi * 32 + (lane & 31);
      a[mi] = *(const bf16x8_t*)&as[r * BK + ((chunk ^ (r & 15)) << 3)];
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) acc[mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi], w, acc[mi], 0, 0, 0);
  };

  // A uniform pipeline over RB_D + 1 weight register sets. Step t waits for tile t, passes the
  // barrier, issues the weight loads of tile t + RB_D, multiplies tile t and then issues the
  // activation loads of tile t + RB_D (past the end: the range's last tile again, into a free
  // stage and set). RB_D weight tiles stay in flight during the multiply, and each wait leaves
  // exactly the RB_D - 1 younger tile groups outstanding. (Activation loads issued before the
  // multiply would make the compiler wait for them before its LDS reads.)
  const int n = ke - kb;
  if (n > 0) {
    bf16x8_t w0[W_INS], w1[W_INS], w2[W_INS], w3[W_INS];
    issue_w(kb, w0);
    issue_a(kb, 0);
    issue_w(kb + min(1, n - 1), w1);
    issue_a(kb + min(1, n - 1), 1);
    issue_w(kb + min(2, n - 1), w2);
    issue_a(kb + min(2, n - 1), 2);
    auto step = [&](int t, bf16x8_t (&w)[W_INS], bf16x8_t (&wnext)[W_INS]) {
      rows_wait_vm<(D - 1) * LPT>();
      // each wave waited for its own loads of tile t; after the barrier the tile is in LDS and
      // every wave is past tile t - 1, whose stage the activation refill below reuses
      asm volatile("s_barrier" ::: "memory");
      const int tnext = kb + min(t + D, n - 1);
      issue_w(tnext, wnext);
      const bf16_t* as = smem + (t % AS) * BM * BK;
#pragma unroll
      for (int j = 0; j < W_INS; ++j) mfma_step(as, lg * 8 + j, w[j]);
      issue_a(tnext, (t + D) % AS);
    };
    // whole groups of four steps in the loop (no conditional step before its back edge, so the
    // compiler's own wait before each multiply counts the younger groups), the rest after it
    int t = 0;
    for (; t + 4 <= n; t += 4) {
      step(t, w0, w3);
      step(t + 1, w1, w0);
      step(t + 2, w2, w1);
      step(t + 3, w3, w2);
    }
    if (t < n) step(t, w0, w3);
    if (t + 1 < n) step(t + 1, w1, w0);
    if (t + 2 < n) step(t + 2, w2, w1);
    rows_wait_vm<0>();
  }

  // acc[mi][r] holds C[row 32 mi + 8 (r >> 2) + 4 lg + (r & 3)][col 32 w + lane % 32].
  const int col = n0 + wid * 32 + (lane & 31);
  if (col >= ncols) return;
  const int64_t wcol = lora_tile ? (int64_t)p.N + col : col;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + mi * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
      if (row >= p.M) continue;
      if constexpr (DIRECT) {
        float v = acc[mi][r];
        if (p.Res) v += bf16_to_f32(p.Res[(int64_t)row * p.ldres + col]);
        p.C[(int64_t)row * p.ldc + col] = f32_to_bf16(v);
      } else {
        p.ws[((int64_t)split * p.M + row) * p.ldw + wcol] = acc[mi][r];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Reduction with the rank-r LoRA update and the epilogue. Workgroup tile: 16 rows x 128 product
// columns ("slots"; EPI 0) or 16 rows x 64 SwiGLU features, i.e. the 64 gate and the 64 matching up
// columns (EPI 1).
//   1. h = bf16(m (.) sum of the LoRA-column partials) for the tile's rows (all R columns) into
//      LDS, and the slots' (s B) rows into LDS;
//   2. the rank-r update u[row, slot] = h[row, seg(slot) + :r] . (s B)[slot, :r] with 16x16x32
//      MFMAs (each wave two 16-slot tiles), fp32 into LDS;
//   3. every thread adds the partials of 4 columns (and 4 up columns) of its rows in range order,
//      then u, the residual, and rounds:
// EPI 0: C[M, N]   = bf16(sum + u + Res);
// EPI 1: C[M, N/2] = bf16(silu(g) * u), g = bf16(gate column value), u = bf16(up column value)
//        (the [gate | up] product rounded to bf16 and then the SwiGLU of unok_swiglu_fwd).
// Segment boundaries are multiples of 16, so each 16-slot tile reads one segment of h.
// ---------------------------------------------------------------------------------------
constexpr int RR_ROWS = 16, RR_SLOTS = 128, RR_ULD = RR_SLOTS + 4;

struct RowsReduce {
  const float* ws; int64_t ldw; int splits;
  int M, N, R;
  const bf16_t* LB; int64_t ldlb; int r;   // [N, r] (s B); null: no LoRA
  int nseg; int seg_end[4]; int seg_col[4];
  const uint8_t* gate;
  const bf16_t* Res; int64_t ldres;
  bf16_t* C; int64_t ldc;
};

__device__ __forceinline__ int red_seg_col(const RowsReduce& p, int n) {
  int c = p.seg_col[0];
  if (p.nseg > 1 && n >= p.seg_end[0]) c = p.seg_col[1];
  if (p.nseg > 2 && n >= p.seg_end[1]) c = p.seg_col[2];
  if (p.nseg > 3 && n >= p.seg_end[2]) c = p.seg_col[3];
  return c;
}

__device__ __forceinline__ int round32(int x) { return (x + 31) & ~31; }

template <int EPI>
__global__ __launch_bounds__(256) void rows_reduce_kernel(const RowsReduce p) {
  constexpr int NH = EPI == 1 ? 2 : 1;             // column groups per thread: (gate, up) or one
  constexpr int NG = RR_SLOTS / (4 * NH);          // column groups of 4 per workgroup row: 32 / 16
  constexpr int RPT = RR_ROWS * NG / 256;          // rows per thread: 2 (EPI 0) or 1 (EPI 1)
  extern __shared__ __attribute__((aligned(16))) float rsm[];
  const bool lora = p.LB != nullptr;
  const int rp = round32(p.r);
  const int hld = p.R + 32;                        // bf16 row stride of h (zero tail read by the last steps)
  const int rld = rp + 8;                          // bf16 row stride of the staged (s B) rows
  float* Us = rsm;                                                   // [RR_ROWS][RR_ULD] fp32
  bf16_t* Hs = (bf16_t*)(rsm + RR_ROWS * RR_ULD);                    // [RR_ROWS][hld]
  bf16_t* Ls = Hs + RR_ROWS * hld;                                   // [RR_SLOTS][rld]

  const int nout = EPI == 1 ? p.N / 2 : p.N;
  const int ctiles = (nout + NG * 4 - 1) / (NG * 4);
  const int r0 = (blockIdx.x / ctiles) * RR_ROWS;
  const int c0 = (blockIdx.x % ctiles) * NG * 4;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t plane = (int64_t)p.M * p.ldw;

  // product column of slot q of this tile: EPI 0: c0 + q; EPI 1: gate c0 + q for q < 64, up
  // N/2 + c0 + q - 64 above
  auto slot_col = [&](int q) {
    if constexpr (EPI == 1) return q < NG * 4 ? c0 + q : nout + c0 + (q - NG * 4);
    else return c0 + q;
  };
  if (lora) {
    // h: four (row, column) items per thread at a time, each with up to eight ranges' loads in flight
    const int items = RR_ROWS * p.R;
    for (int i0 = tid; i0 < items; i0 += 4 * 256) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      const float* src[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = min(i0 + u * 256, items - 1);
        const int row = min(r0 + i / p.R, p.M - 1);
        src[u] = p.ws + (int64_t)row * p.ldw + p.N + i % p.R;
      }
      for (int k0 = 0; k0 < p.splits; k0 += 8) {
        float v[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int q = 0; q < 8; ++q) v[u][q] = k0 + q < p.splits ? src[u][(k0 + q) * plane] : 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (k0 + q < p.splits) acc[u] += v[u][q];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * 256;
        if (i >= items) break;
        const int rr = i / p.R, j = i % p.R;
        const int row = min(r0 + rr, p.M - 1);
        const bool on = p.gate == nullptr || p.gate[row] != 0;
        Hs[rr * hld + j] = on ? f32_to_bf16(acc[u]) : (bf16_t)0;
      }
    }
    for (int i = tid; i < RR_ROWS * 32; i += 256) Hs[(i / 32) * hld + p.R + i % 32] = 0;
    const int vec = p.r / 8;
    for (int i = tid; i < RR_SLOTS * vec; i += 256) {
      const int q = i / vec, v = i % vec;
      const int colq = min(slot_col(q), p.N - 1);
      *(uint4*)(Ls + q * rld + v * 8) = *(const uint4*)(p.LB + (int64_t)colq * p.ldlb + v * 8);
    }
    __syncthreads();
    // rank-r update on MFMA: wave w takes slot tiles 2 w and 2 w + 1; lane l supplies (s B) of slot
    // l % 16 and h of row l % 16 at k = 32 kk + 8 (l / 16) + [0, 8); the result of slot
    // 4 (l / 16) + e, row l % 16 is D element e of lane l
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int s0 = (wid * 2 + tt) * 16;
      const int hc = red_seg_col(p, slot_col(s0));
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
      for (int kk = 0; kk < rp; kk += 32) {
        const int k = kk + 8 * (lane >> 4);
        bf16x8_t lb = *(const bf16x8_t*)(Ls + (s0 + (lane & 15)) * rld + k);
        if (k >= p.r) lb = __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
        const bf16x8_t hv = *(const bf16x8_t*)(Hs + (lane & 15) * hld + hc + k);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lb, hv, d, 0, 0, 0);
      }
      *(f32x4_t*)(Us + (lane & 15) * RR_ULD + s0 + 4 * (lane >> 4)) = d;
    }
    __syncthreads();
  }

  const int cg = tid % NG, rg = tid / NG;
  const int cbase = c0 + cg * 4;
  if (cbase >= nout) return;
  // partial sums: all rows and column groups of this thread, up to eight ranges in flight each,
  // added in range order
  float4 acc[RPT][NH];
  const float4* src[RPT][NH];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int row = min(r0 + rg * RPT + i, p.M - 1);
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      acc[i][h] = make_float4(0.f, 0.f, 0.f, 0.f);
      src[i][h] = (const float4*)(p.ws + (int64_t)row * p.ldw + cbase + h * nout);
    }
  }
  const int64_t plane4 = plane / 4;
  for (int k0 = 0; k0 < p.splits; k0 += 8) {
    float4 v[RPT][NH][8];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int q = 0; q < 8; ++q)
          v[i][h][q] = k0 + q < p.splits ? src[i][h][(k0 + q) * plane4] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (k0 + q < p.splits) acc[i][h] += v[i][h][q];
  }
  if (lora) {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int h = 0; h < NH; ++h) acc[i][h] += *(const float4*)(Us + (rg * RPT + i) * RR_ULD + h * NG * 4 + cg * 4);
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int row = r0 + rg * RPT + i;
    if (row >= p.M) continue;
    const float a[4] = {acc[i][0].x, acc[i][0].y, acc[i][0].z, acc[i][0].w};
    float o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if constexpr (EPI == 0) {
        float v = a[c];
        if (p.Res) v += bf16_to_f32(p.Res[(int64_t)row * p.ldres + cbase + c]);
        o[c] = v;
      } else {
        const float b[4] = {acc[i][NH - 1].x, acc[i][NH - 1].y, acc[i][NH - 1].z, acc[i][NH - 1].w};
        const float g = Elem<bf16_t>::round(a[c]);
        const float u = Elem<bf16_t>::round(b[c]);
        o[c] = g * sigmoidf_(g) * u;
      }
    }
    uint2 packed;
    packed.x = pack2_bf16(o[0], o[1]);
    packed.y = pack2_bf16(o[2], o[3]);
    *(uint2*)(p.C + (int64_t)row * p.ldc + cbase) = packed;
  }
}

// K ranges for an M x N product (plus R LoRA columns) of nk K tiles: the count that minimises the
// critical path in tile steps (waves of 256 workgroups, one per CU, times the K tiles of the
// longest range plus two for the pipeline fill), the partial-sum traffic (written and read once,
// priced at half a weight tile step per 32 KB per CU because it stays in the on-chip caches for
// these sizes) and the reduction's serial loads (a quarter step per range).
int rows_auto_splits(int M, int N, int R, int nk, bool need_ws) {
  const int64_t tiles = (int64_t)((M + RB_M - 1) / RB_M) * ((N + RB_N - 1) / RB_N + (R + RB_N - 1) / RB_N);
  int best = 1;
  double best_t = 1e30;
  const int smax = nk < 64 ? nk : 64;
  for (int s = 1; s <= smax; ++s) {
    const int64_t wgs = tiles * s;
    const double waves = (double)((wgs + 255) / 256);
    const double steps = waves * (double)((nk + s - 1) / s + 2) + 0.25 * s;
    const double part = (s > 1 || need_ws) ? 0.5 * (double)s * M * (N + R) * 8.0 / (256.0 * 32768.0) : 0.0;
    const double t = steps + part;
    if (t < best_t - 1e-9) { best_t = t; best = s; }
  }
  return best;
}

bool rows_needs_ws(int epilogue, int R, int splits) { return splits > 1 || epilogue != 0 || R > 0; }

size_t rows_reduce_lds(int R, int r) {
  if (R == 0) return 0;
  const int rp = (r + 31) & ~31;
  return (size_t)RR_ROWS * RR_ULD * sizeof(float) + (size_t)RR_ROWS * (R + 32) * sizeof(bf16_t) +
         (size_t)RR_SLOTS * (rp + 8) * sizeof(bf16_t);
}

// ---------------------------------------------------------------------------------------
// Attention of a draft block over the KV cache, in three kernels per layer:
//   prep     q/k RMSNorm + RoPE of the fused qkv rows (the arithmetic of unok_qknorm_rope_fwd),
//            the block's K and V rows into the caches at (b, kv head, length_b + t), and the
//            queries into the decode layout: the queries of one (sequence, K/V head) pair, rep q
//            heads x L rows, are the first rep * L of 128 rows (row 128 pair + L (h % rep) + t),
//            the rest zero;
//   attn     unok_attn_fwd_split over S key ranges of each pair's cache rows;
//   combine  the S partial rows of each query merged by their log-sum-exp weights and written to
//            the attention output [B * L, nq * D] at (b * L + t, head h).
// ---------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void decode_prep_kernel(const bf16_t* __restrict__ qkv, int64_t ld,
                                                          const bf16_t* __restrict__ wq, const bf16_t* __restrict__ wk,
                                                          const int64_t* __restrict__ lengths,
                                                          const float* __restrict__ inv_freq, float eps,
                                                          bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
                                                          int max_len, bf16_t* __restrict__ qd, int B, int L, int nq,
                                                          int nk) {
  constexpr int LPH = D / 8, HALF = D / 2;          // lanes per head row, 8 elements per lane
  const int lane = threadIdx.x & 63;
  const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPH;
  const int sub = lane % LPH, c0 = sub * 8;
  const int M = B * L, nh = nq + 2 * nk, rep = nq / nk;
  const int64_t heads = (int64_t)M * nh;
  const int pad = 128 - rep * L;
  if (item >= heads) {
    // zero padding rows of the decode query layout
    const int64_t z = item - heads;
    if (z >= (int64_t)B * nk * pad) return;
    const int64_t row = (z / pad) * 128 + rep * L + z % pad;
    *(uint4*)(qd + row * D + c0) = make_uint4(0, 0, 0, 0);
    return;
  }
  const int m = (int)(item / nh), hd = (int)(item % nh);
  const int b = m / L, t = m % L;
  const int64_t len = lengths[b];
  float x[8];
  {
    const uint4 u = *(const uint4*)(qkv + (int64_t)m * ld + (int64_t)hd * D + c0);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[2 * i] = __uint_as_float(w[i] << 16); x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u); }
  }
  bf16_t* dst;
  if (hd < nq + nk) {
    const bool isq = hd < nq;
    const bf16_t* wn = isq ? wq : wk;
    if (wn != nullptr) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
#pragma unroll
      for (int o = LPH / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
      const float r = rsqrtf(ss / (float)D + eps);
      const uint4 u = *(const uint4*)(wn + c0);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float w0 = __uint_as_float(w[i] << 16), w1 = __uint_as_float(w[i] & 0xffff0000u);
        x[2 * i] = x[2 * i] * r * w0;
        x[2 * i + 1] = x[2 * i + 1] * r * w1;
      }
    }
    const float p = (float)(len + t);
    const int j0 = c0 % HALF;
    const float sgn = c0 < HALF ? -1.f : 1.f;
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float sv, cv;
      sincosf(p * inv_freq[j0 + e], &sv, &cv);
      const float y = __shfl_xor(x[e], LPH / 2, 64);   // partner element i +- d/2
      out[e] = x[e] * cv + sgn * y * sv;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = out[e];
    if (isq) {
      const int kv = hd / rep, rr = hd % rep;
      dst = qd + ((int64_t)(b * nk + kv) * 128 + rr * L + t) * D;
    } else {
      if (len + t >= max_len) return;
      dst = kc + ((int64_t)(b * nk + hd - nq) * max_len + len + t) * D;
    }
  } else {
    if (len + t >= max_len) return;
    dst = vc + ((int64_t)(b * nk + hd - nq - nk) * max_len + len + t) * D;
  }
  *(uint4*)(dst + c0) = make_uint4(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]), pack2_bf16(x[4], x[5]),
                                   pack2_bf16(x[6], x[7]));
}

// O[dst[i]] = sum_s 2^(lse_s - m) O_s[i] / sum_s 2^(lse_s - m) over the S partial rows s * QR + i
// (lse in log2 units, m their maximum; a range without keys has lse = -inf and weight 0); rows
// with dst[i] < 0 are skipped.
template <int D>
__global__ __launch_bounds__(256) void attn_split_combine_kernel(const bf16_t* __restrict__ op, int64_t ldp,
                                                                 const float* __restrict__ lse,
                                                                 const int32_t* __restrict__ dst, int QR, int S,
                                                                 bf16_t* __restrict__ out, int64_t ldo) {
  constexpr int LPR = D / 8;
  const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
  if (item >= QR) return;
  const int i = (int)item, c0 = (threadIdx.x % LPR) * 8;
  const int d = dst[i];
  if (d < 0) return;
  float m = -INFINITY;
  for (int s = 0; s < S; ++s) m = fmaxf(m, lse[(int64_t)s * QR + i]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (m != -INFINITY) {
    for (int s = 0; s < S; ++s) {
      const float l = lse[(int64_t)s * QR + i];
      if (l == -INFINITY) continue;
      const float w = exp2f(l - m);
      wsum += w;
      const uint4 u = *(const uint4*)(op + ((int64_t)s * QR + i) * ldp + c0);
      const uint32_t v[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[2 * k] += w * __uint_as_float(v[k] << 16);
        acc[2 * k + 1] += w * __uint_as_float(v[k] & 0xffff0000u);
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  *(uint4*)(out + (int64_t)d * ldo + c0) =
      make_uint4(pack2_bf16(acc[0] * inv, acc[1] * inv), pack2_bf16(acc[2] * inv, acc[3] * inv),
                 pack2_bf16(acc[4] * inv, acc[5] * inv), pack2_bf16(acc[6] * inv, acc[7] * inv));
}

}  // namespace

// Workspace bytes of unok_gemm_nt_rows for this shape (R = 0 without LoRA; splits <= 0: the
// automatic count).
UNOK_EXPORT int64_t unok_gemm_nt_rows_workspace(int M, int N, int K, int R, int epilogue, int splits) {
  if (M <= 0 || N <= 0 || K <= 0 || R < 0) return 0;
  const int nk = K / RB_K;
  const int s = splits > 0 ? splits : rows_auto_splits(M, N, R, nk > 0 ? nk : 1, epilogue != 0 || R > 0);
  if (!rows_needs_ws(epilogue, R, s)) return 0;
  return (int64_t)s * M * (N + R) * (int64_t)sizeof(float);
}

UNOK_EXPORT int unok_gemm_nt_rows(int M, int N, int K, const void* A, int64_t lda, const void* B, int64_t ldb,
                                  const void* LA, int64_t ldla, int R, const void* LB, int64_t ldlb, int r,
                                  int nseg, const int* seg_end, const int* seg_col,
                                  void* C, int64_t ldc, const void* Res, int64_t ldres, const uint8_t* gate,
                                  int epilogue, int splits, void* workspace, int64_t ws_bytes, void* stream) {
  UNOK_REQUIRE(M >= 0 && N >= 0 && K >= 0, UNOK_EINVAL, "gemm_nt_rows: negative size M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return 0;
  UNOK_REQUIRE(epilogue == 0 || epilogue == 1, UNOK_EINVAL, "gemm_nt_rows: epilogue %d is not 0 or 1", epilogue);
  UNOK_REQUIRE(K > 0 && K % RB_K == 0, UNOK_EINVAL, "gemm_nt_rows: K=%d must be a positive multiple of 128", K);
  UNOK_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0, UNOK_EALIGN,
               "gemm_nt_rows: lda=%lld ldb=%lld must be multiples of 8 and A/B 16-byte aligned", (long long)lda,
               (long long)ldb);
  UNOK_REQUIRE(N % 4 == 0 && ldc % 4 == 0 && ((uintptr_t)C & 7) == 0, UNOK_EALIGN,
               "gemm_nt_rows: N=%d and ldc=%lld must be multiples of 4 and C 8-byte aligned", N, (long long)ldc);
  UNOK_REQUIRE(epilogue == 0 || N % 32 == 0, UNOK_EINVAL, "gemm_nt_rows: the SwiGLU epilogue needs N=%d a multiple of 32",
               N);
  UNOK_REQUIRE(epilogue == 0 || Res == nullptr, UNOK_EINVAL, "gemm_nt_rows: the SwiGLU epilogue takes no residual");
  UNOK_REQUIRE(Res == nullptr || (ldres % 4 == 0 && ((uintptr_t)Res & 7) == 0), UNOK_EALIGN,
               "gemm_nt_rows: ldres=%lld must be a multiple of 4 and Res 8-byte aligned", (long long)ldres);
  const bool lora = LA != nullptr;
  RowsReduce q{};
  q.nseg = 1;
  for (int i = 0; i < 4; ++i) { q.seg_end[i] = N; q.seg_col[i] = 0; }
  if (lora) {
    UNOK_REQUIRE(R > 0 && R <= 512 && R % 8 == 0 && LB != nullptr && r > 0 && r <= 128 && r % 8 == 0, UNOK_EINVAL,
                 "gemm_nt_rows: LoRA needs 0 < R <= 512 A rows (a multiple of 8) and a rank 0 < r <= 128 "
                 "(a multiple of 8), got R=%d r=%d", R, r);
    UNOK_REQUIRE(ldla % 8 == 0 && ((uintptr_t)LA & 15) == 0 && ldlb % 8 == 0 && ((uintptr_t)LB & 15) == 0,
                 UNOK_EALIGN, "gemm_nt_rows: ldla=%lld ldlb=%lld must be multiples of 8 and LA/LB 16-byte aligned",
                 (long long)ldla, (long long)ldlb);
    if (nseg > 0) {
      UNOK_REQUIRE(nseg <= 4 && seg_end && seg_col, UNOK_EINVAL, "gemm_nt_rows: at most 4 segments");
      q.nseg = nseg;
      for (int i = 0; i < nseg; ++i) {
        q.seg_end[i] = seg_end[i];
        q.seg_col[i] = seg_col[i];
        UNOK_REQUIRE(seg_col[i] >= 0 && seg_col[i] % 8 == 0 && seg_col[i] + r <= R, UNOK_EINVAL,
                     "gemm_nt_rows: segment %d reads LoRA hidden columns %d..%d of %d (start a multiple of 8)", i, seg_col[i],
                     seg_col[i] + r, R);
        UNOK_REQUIRE(i + 1 == nseg || seg_end[i] % 16 == 0, UNOK_EINVAL,
                     "gemm_nt_rows: segment end %d not a multiple of 16", seg_end[i]);
      }
      UNOK_REQUIRE(seg_end[nseg - 1] == N, UNOK_EINVAL, "gemm_nt_rows: last segment must end at N");
    } else {
      UNOK_REQUIRE(r <= R, UNOK_EINVAL, "gemm_nt_rows: rank %d exceeds the %d LoRA A rows", r, R);
    }
  } else {
    R = 0;
  }
  const int nk = K / RB_K;
  const int s = splits > 0 ? splits : rows_auto_splits(M, N, R, nk, epilogue != 0 || lora);
  UNOK_REQUIRE(s <= nk, UNOK_EINVAL, "gemm_nt_rows: %d K ranges for %d K tiles", s, nk);

  RowsGemm p{};
  p.A = (const bf16_t*)A; p.lda = lda;
  p.B = (const bf16_t*)B; p.ldb = ldb;
  p.LA = lora ? (const bf16_t*)LA : nullptr; p.ldla = ldla;
  p.M = M; p.N = N; p.K = K; p.R = R;
  p.splits = s;
  const int64_t ntiles = (int64_t)((N + RB_N - 1) / RB_N) + (lora ? (R + RB_N - 1) / RB_N : 0);
  const int64_t nb = (int64_t)((M + RB_M - 1) / RB_M) * ntiles * s;
  UNOK_REQUIRE(nb < (1ll << 31), UNOK_EINVAL, "gemm_nt_rows: grid too large");
  constexpr size_t lds = (size_t)(RB_D + 1) * RB_M * RB_K * sizeof(bf16_t);
  hipStream_t st = (hipStream_t)stream;
  if (!rows_needs_ws(epilogue, R, s)) {
    p.C = (bf16_t*)C; p.ldc = ldc; p.Res = (const bf16_t*)Res; p.ldres = ldres;
    UNOK_SET_LDS_ONCE((gemm_nt_rows_kernel<true>), lds);
    hipLaunchKernelGGL((gemm_nt_rows_kernel<true>), dim3((unsigned)nb), dim3(RB_W * 64), lds, st, p);
    return unok::check_launch("gemm_nt_rows");
  }
  const int64_t need = (int64_t)s * M * (N + R) * (int64_t)sizeof(float);
  UNOK_REQUIRE(workspace != nullptr && ws_bytes >= need && ((uintptr_t)workspace & 15) == 0, UNOK_EINVAL,
               "gemm_nt_rows: workspace of %lld bytes (16-byte aligned) required, got %lld", (long long)need,
               (long long)ws_bytes);
  p.ws = (float*)workspace; p.ldw = N + R;
  UNOK_SET_LDS_ONCE((gemm_nt_rows_kernel<false>), lds);
  hipLaunchKernelGGL((gemm_nt_rows_kernel<false>), dim3((unsigned)nb), dim3(RB_W * 64), lds, st, p);
  int rc = unok::check_launch("gemm_nt_rows");
  if (rc) return rc;

  q.ws = (const float*)workspace; q.ldw = N + R; q.splits = s;
  q.M = M; q.N = N; q.R = R;
  q.LB = lora ? (const bf16_t*)LB : nullptr; q.ldlb = ldlb; q.r = lora ? r : 0;
  q.gate = gate;
  q.Res = (const bf16_t*)Res; q.ldres = ldres;
  q.C = (bf16_t*)C; q.ldc = ldc;
  const int nout = epilogue == 1 ? N / 2 : N;
  const int cw = epilogue == 1 ? RR_SLOTS / 2 : RR_SLOTS;
  const int64_t blocks = (int64_t)((M + RR_ROWS - 1) / RR_ROWS) * ((nout + cw - 1) / cw);
  const size_t rlds = rows_reduce_lds(R, q.r);
  if (epilogue == 0) {
    UNOK_SET_LDS_ONCE((rows_reduce_kernel<0>), 96 * 1024);
    hipLaunchKernelGGL((rows_reduce_kernel<0>), dim3((unsigned)blocks), dim3(256), rlds, st, q);
  } else {
    UNOK_SET_LDS_ONCE((rows_reduce_kernel<1>), 96 * 1024);
    hipLaunchKernelGGL((rows_reduce_kernel<1>), dim3((unsigned)blocks), dim3(256), rlds, st, q);
  }
  return unok::check_launch("gemm_nt_rows_reduce");
}

// q/k norm + RoPE of a draft block's fused qkv rows, its K/V rows into the caches and its queries
// into the decode layout (see decode_prep_kernel). bf16; D in {64, 128}; wq / wk null: no q/k norm.
UNOK_EXPORT int unok_decode_prep(int B, int L, int nq, int nk, int D, const void* qkv, int64_t ld, const void* wq,
                                 const void* wk, const int64_t* lengths, const float* inv_freq, float eps, void* kc,
                                 void* vc, int max_len, void* qd, void* stream) {
  UNOK_REQUIRE(B >= 0 && L >= 0 && nq > 0 && nk > 0 && nq % nk == 0, UNOK_EINVAL,
               "decode_prep: B=%d L=%d nq=%d nk=%d", B, L, nq, nk);
  if (B == 0 || L == 0) return 0;
  UNOK_REQUIRE(D == 64 || D == 128, UNOK_EINVAL, "decode_prep: head dim %d not in {64,128}", D);
  UNOK_REQUIRE((nq / nk) * L <= 128, UNOK_EINVAL, "decode_prep: %d q heads x %d rows exceed 128 rows per K/V head",
               nq / nk, L);
  UNOK_REQUIRE(ld % 8 == 0 && ((uintptr_t)qkv & 15) == 0 && ((uintptr_t)kc & 15) == 0 && ((uintptr_t)vc & 15) == 0 &&
                   ((uintptr_t)qd & 15) == 0 && (wq == nullptr || ((uintptr_t)wq & 15) == 0) &&
                   (wk == nullptr || ((uintptr_t)wk & 15) == 0),
               UNOK_EALIGN, "decode_prep: rows must be 16-byte aligned");
  const int64_t heads = (int64_t)B * L * (nq + 2 * nk);
  const int64_t pads = (int64_t)B * nk * (128 - (nq / nk) * L);
  const int lph = D / 8;
  const int64_t blocks = ((heads + pads) * lph + 255) / 256;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128)
    hipLaunchKernelGGL((decode_prep_kernel<128>), dim3((unsigned)blocks), dim3(256), 0, st, (const bf16_t*)qkv, ld,
                       (const bf16_t*)wq, (const bf16_t*)wk, lengths, inv_freq, eps, (bf16_t*)kc, (bf16_t*)vc, max_len,
                       (bf16_t*)qd, B, L, nq, nk);
  else
    hipLaunchKernelGGL((decode_prep_kernel<64>), dim3((unsigned)blocks), dim3(256), 0, st, (const bf16_t*)qkv, ld,
                       (const bf16_t*)wq, (const bf16_t*)wk, lengths, inv_freq, eps, (bf16_t*)kc, (bf16_t*)vc, max_len,
                       (bf16_t*)qd, B, L, nq, nk);
  return unok::check_launch("decode_prep");
}

// Merge of the S partial rows of split-key attention (see attn_split_combine_kernel). bf16.
UNOK_EXPORT int unok_attn_split_combine(int QR, int S, int D, const void* opart, int64_t ldp, const float* lse,
                                        const int32_t* dst, void* out, int64_t ldo, void* stream) {
  UNOK_REQUIRE(QR >= 0 && S >= 1, UNOK_EINVAL, "attn_split_combine: QR=%d S=%d", QR, S);
  if (QR == 0) return 0;
  UNOK_REQUIRE(D == 64 || D == 128, UNOK_EINVAL, "attn_split_combine: head dim %d not in {64,128}", D);
  UNOK_REQUIRE(ldp % 8 == 0 && ldo % 8 == 0 && ((uintptr_t)opart & 15) == 0 && ((uintptr_t)out & 15) == 0, UNOK_EALIGN,
               "attn_split_combine: rows must be 16-byte aligned");
  const int64_t blocks = ((int64_t)QR * (D / 8) + 255) / 256;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128)
    hipLaunchKernelGGL((attn_split_combine_kernel<128>), dim3((unsigned)blocks), dim3(256), 0, st,
                       (const bf16_t*)opart, ldp, lse, dst, QR, S, (bf16_t*)out, ldo);
  else
    hipLaunchKernelGGL((attn_split_combine_kernel<64>), dim3((unsigned)blocks), dim3(256), 0, st,
                       (const bf16_t*)opart, ldp, lse, dst, QR, S, (bf16_t*)out, ldo);
  return unok::check_launch("attn_split_combine");
}
