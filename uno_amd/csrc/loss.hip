// Objective kernels over LM-head logits.
//
// Cross-entropy (training/trainer.py:267-283): the LM head is evaluated in vocabulary chunks
// (GEMM into a chunk buffer); row_lse_update merges each chunk into a running (max, sum-exp)
// per row and captures the target logit, so the full [rows x vocab] logits never exist.
// The backward recomputes each chunk and writes dz = g * w * (softmax - onehot) for the
// data-gradient GEMM. Row weights w = 1 / p_mask; the 1 / max(token_count, 1) normaliser and
// the upstream gradient come as device scalars (no host synchronisation).
//
// Total variation (training/losses.py:76-183) and reverse KL (losses.py:59-73) run over
// materialised logits with fp32 per-row statistics, matching the reference's per-chunk fp32
// math; TV's gradient is p * (sign(p - q) - sum sign * p) with sign(0) = 0.
#include "common.h"

#include <type_traits>

// Floating-point contraction is off in this file: TV must see d = p - q == 0 exactly when
// p == q (sign(0) = 0), which a fused multiply-add of p's scaling into the subtraction breaks.
#pragma clang fp contract(off)

template <typename T> __device__ __forceinline__ float ldf(const T* p) { return Elem<T>::load(p); }

// 16 bytes of a row as floats: 8 bf16 or 4 fp32 values.
template <typename T> constexpr int VN16 = 16 / (int)sizeof(T);
template <typename T> __device__ __forceinline__ void ld16(const T* p, float (&v)[VN16<T>]) {
  const uint4 u = *(const uint4*)p;
  if constexpr (std::is_same<T, float>::value) {
    v[0] = __uint_as_float(u.x); v[1] = __uint_as_float(u.y); v[2] = __uint_as_float(u.z); v[3] = __uint_as_float(u.w);
  } else {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = __uint_as_float(w[i] << 16); v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u); }
  }
}
template <typename T> __device__ __forceinline__ void st16(T* p, const float (&v)[VN16<T>]) {
  if constexpr (std::is_same<T, float>::value) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    *(uint4*)p = make_uint4(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]), pack2_bf16(v[4], v[5]), pack2_bf16(v[6], v[7]));
  }
}
// The row kernels below walk a row 16 bytes per thread and step when every row pointer involved
// is 16-byte aligned, and the rest of the row (or a misaligned row) one element per thread.
__device__ __forceinline__ bool al16p(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Running softmax statistics of a logits chunk z[R, Vc] (columns c0..c0+Vc of the vocab).
// One pass over the row: each thread keeps its own (max, sum-exp), rescaled when its max grows,
// with 16-byte loads for fp32 rows that allow them; the block then merges the pairs.
template <typename T>
__global__ __launch_bounds__(256) void row_lse_update_kernel(const T* __restrict__ z, int64_t ldz, int Vc, int c0,
                                                             const int64_t* __restrict__ tgt, float* run_max,
                                                             float* run_sum, float* zt, int first) {
  __shared__ float red[32];
  const int row = blockIdx.x;
  const T* zr = z + (int64_t)row * ldz;
  float m = -INFINITY, s = 0.f;
  // A -inf value adds nothing; skipping it also keeps exp(-inf - -inf) = NaN out of the sum while
  // this thread has seen nothing else.
  auto add = [&](float v) {
    if (v > m) { s = s * fast_expf(m - v) + 1.f; m = v; }   // fast_expf(-inf) = 0 on the first value
    else if (v != -INFINITY) s += fast_expf(v - m);
  };
  int j0 = 0;
  if constexpr (std::is_same<T, float>::value) {
    if (((uintptr_t)zr & 15) == 0) {
      const int nv = Vc / 4;
      for (int q = threadIdx.x; q < nv; q += 256) {
        const float4 v = *(const float4*)(zr + 4 * q);
        const float mv = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
        if (mv == -INFINITY) continue;   // four -inf values add nothing
        if (mv > m) { s *= fast_expf(m - mv); m = mv; }
        s += fast_expf(v.x - m) + fast_expf(v.y - m) + fast_expf(v.z - m) + fast_expf(v.w - m);
      }
      j0 = 4 * nv;
    }
  }
  for (int j = j0 + threadIdx.x; j < Vc; j += 256) add(ldf(zr + j));
  const float mb = block_max(m, red);
  s = block_sum(m == -INFINITY ? 0.f : s * fast_expf(m - mb), red);
  m = mb;
  if (threadIdx.x == 0) {
    float M0 = first ? -INFINITY : run_max[row];
    float S0 = first ? 0.f : run_sum[row];
    const float Mn = fmaxf(M0, m);
    run_sum[row] = (S0 > 0.f ? S0 * fast_expf(M0 - Mn) : 0.f) + s * fast_expf(m - Mn);
    run_max[row] = Mn;
    if (tgt) {
      const int64_t t = tgt[row];
      if (t >= c0 && t < c0 + Vc) zt[row] = ldf(zr + (t - c0));
    }
  }
}

// (v, i) beats (bv, bi) under torch.argmax's order: NaN above every number, then larger values,
// then the smaller index among equal values (first occurrence).
__device__ __forceinline__ bool argmax_beats(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// First-index argmax merge over a chunk: best (value, index) per row.
template <typename T>
__global__ __launch_bounds__(256) void row_argmax_update_kernel(const T* __restrict__ z, int64_t ldz, int Vc, int c0,
                                                                float* best_val, int64_t* best_idx, int first) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int row = blockIdx.x;
  const T* zr = z + (int64_t)row * ldz;
  float bv = -INFINITY;
  int bi = INT_MAX;                      // INT_MAX: this thread has seen no element
  auto take = [&](float v, int j) {
    if (bi == INT_MAX || argmax_beats(v, j, bv, bi)) { bv = v; bi = j; }
  };
  // 16 bytes per thread and step (each thread still visits its columns in increasing order, and
  // the merge below orders ties by column, so the result is the element-wise walk's)
  int j0 = 0;
  if (al16p(zr)) {
    constexpr int VN = VN16<T>;
    const int nv = Vc / VN;
    for (int q = threadIdx.x; q < nv; q += 256) {
      float v[VN];
      ld16(zr + q * VN, v);
#pragma unroll
      for (int e = 0; e < VN; ++e) take(v[e], q * VN + e);
    }
    j0 = nv * VN;
  }
  for (int j = j0 + threadIdx.x; j < Vc; j += 256) take(ldf(zr + j), j);
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      const float v2 = sv[threadIdx.x + o];
      const int i2 = si[threadIdx.x + o];
      if (i2 != INT_MAX && (si[threadIdx.x] == INT_MAX || argmax_beats(v2, i2, sv[threadIdx.x], si[threadIdx.x]))) {
        sv[threadIdx.x] = v2;
        si[threadIdx.x] = i2;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && si[0] != INT_MAX) {
    const float v = sv[0];
    const int64_t idx = (int64_t)si[0] + c0;
    // chunks arrive in increasing column order, so an equal value of a later chunk never wins
    if (first || argmax_beats(v, idx, best_val[row], best_idx[row])) { best_val[row] = v; best_idx[row] = idx; }
  }
}

// loss = sum_r w[r] * (lse[r] - zt[r]) * inv_n ; also stores lse. Single workgroup, fixed order.
__global__ __launch_bounds__(1024) void ce_finish_kernel(int R, const float* run_max, const float* run_sum,
                                                         const float* zt, const float* w, const float* inv_n,
                                                         float* lse, float* loss) {
  __shared__ float red[32];
  float acc = 0.f;
  for (int r = threadIdx.x; r < R; r += 1024) {
    const float l = run_max[r] + logf(run_sum[r]);
    lse[r] = l;
    acc += (w ? w[r] : 1.f) * (l - zt[r]);
  }
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) loss[0] = acc * (inv_n ? inv_n[0] : 1.f);
}

// dz[r, j] = g * inv_n * w[r] * (exp(z - lse[r]) - [c0 + j == tgt[r]])
template <typename TO>
__global__ __launch_bounds__(256) void ce_grad_chunk_kernel(const float* __restrict__ z, int64_t ldz, int Vc, int c0,
                                                            const float* __restrict__ lse,
                                                            const int64_t* __restrict__ tgt,
                                                            const float* __restrict__ w, const float* gscale,
                                                            const float* inv_n, TO* __restrict__ dz, int64_t lddz) {
  const int row = blockIdx.x;
  const float l = lse[row];
  const float c = gscale[0] * (inv_n ? inv_n[0] : 1.f) * (w ? w[row] : 1.f);
  const int64_t t = tgt[row] - c0;
  const float* zr = z + (int64_t)row * ldz;
  TO* dr = dz + (int64_t)row * lddz;
  int j0 = 0;
  if constexpr (std::is_same<TO, bf16_t>::value) {
    if (((uintptr_t)zr & 15) == 0 && ((uintptr_t)dr & 7) == 0) {   // 4 logits in, 4 gradients out per load
      const int nv = Vc / 4;
      for (int q = threadIdx.x; q < nv; q += 256) {
        const float4 v = *(const float4*)(zr + 4 * q);
        float p[4] = {fast_expf(v.x - l), fast_expf(v.y - l), fast_expf(v.z - l), fast_expf(v.w - l)};
        if (t >= 4 * q && t < 4 * q + 4) p[t - 4 * q] -= 1.f;
        *(uint2*)(dr + 4 * q) = make_uint2(pack2_bf16(c * p[0], c * p[1]), pack2_bf16(c * p[2], c * p[3]));
      }
      j0 = 4 * nv;
    }
  }
  for (int j = j0 + threadIdx.x; j < Vc; j += 256) {
    float p = fast_expf(zr[j] - l);
    if (j == t) p -= 1.f;
    Elem<TO>::store(dr + j, c * p);
  }
}

// Per-row max and sum-exp over full rows (fp32 statistics).
template <typename T>
__global__ __launch_bounds__(256) void softmax_stats_kernel(const T* __restrict__ z, int64_t ldz, int V, float* mx,
                                                            float* se) {
  __shared__ float red[32];
  constexpr int VN = VN16<T>;
  const int row = blockIdx.x;
  const T* zr = z + (int64_t)row * ldz;
  // One pass: each thread keeps its own (max, sum-exp), rescaled when its max grows, over 16-byte
  // loads; the block then merges the pairs.
  float m = -INFINITY, s = 0.f;
  int j0 = 0;
  if (al16p(zr)) {
    const int nv = V / VN;
    for (int q = threadIdx.x; q < nv; q += 256) {
      float v[VN];
      ld16(zr + q * VN, v);
      float mv = v[0];
#pragma unroll
      for (int e = 1; e < VN; ++e) mv = fmaxf(mv, v[e]);
      if (mv == -INFINITY) continue;   // a group of -inf values adds nothing (and m may still be -inf)
      if (mv > m) { s *= fast_expf(m - mv); m = mv; }
#pragma unroll
      for (int e = 0; e < VN; ++e) s += fast_expf(v[e] - m);
    }
    j0 = nv * VN;
  }
  for (int j = j0 + threadIdx.x; j < V; j += 256) {
    const float v = ldf(zr + j);
    if (v > m) { s = s * fast_expf(m - v) + 1.f; m = v; }   // fast_expf(-inf) = 0 on the first value
    else if (v != -INFINITY) s += fast_expf(v - m);
  }
  const float mb = block_max(m, red);
  s = block_sum(m == -INFINITY ? 0.f : s * fast_expf(m - mb), red);
  if (threadIdx.x == 0) { mx[row] = mb; se[row] = fmaxf(s, 1.17549435e-38f); }
}

// TV forward: row_l1 = sum |ps - pt|, row_S = sum sign(ps - pt) * ps.
template <typename T>
__global__ __launch_bounds__(256) void tv_fwd_kernel(const T* __restrict__ zs, int64_t lds, const T* __restrict__ zt,
                                                     int64_t ldt, int V, const float* ms, const float* ss,
                                                     const float* mt, const float* st, float* row_l1, float* row_S) {
  __shared__ float red[32];
  const int row = blockIdx.x;
  const float a = ms[row], ia = 1.f / ss[row], b = mt[row], ib = 1.f / st[row];
  const T* s = zs + (int64_t)row * lds;
  const T* t = zt + (int64_t)row * ldt;
  float l1 = 0.f, S = 0.f;
  auto elem = [&](float zsv, float ztv) {
    const float ps = fast_expf(zsv - a) * ia, pt = fast_expf(ztv - b) * ib;
    const float d = ps - pt;
    l1 += fabsf(d);
    S += (d > 0.f ? ps : (d < 0.f ? -ps : 0.f));
  };
  int j0 = 0;
  if (al16p(s) && al16p(t)) {
    constexpr int VN = VN16<T>;
    const int nv = V / VN;
    for (int q = threadIdx.x; q < nv; q += 256) {
      float vs[VN], vt[VN];
      ld16(s + q * VN, vs);
      ld16(t + q * VN, vt);
#pragma unroll
      for (int e = 0; e < VN; ++e) elem(vs[e], vt[e]);
    }
    j0 = nv * VN;
  }
  for (int j = j0 + threadIdx.x; j < V; j += 256) elem(ldf(s + j), ldf(t + j));
  l1 = block_sum(l1, red);
  S = block_sum(S, red);
  if (threadIdx.x == 0) { row_l1[row] = l1; row_S[row] = S; }
}

// TV backward: grad[j] = ps_j * (sign_j - S) * g * inv_n; grad may alias zs.
template <typename T>
__global__ __launch_bounds__(256) void tv_bwd_kernel(const T* zs, int64_t lds, const T* __restrict__ zt, int64_t ldt,
                                                     int V, const float* ms, const float* ss, const float* mt,
                                                     const float* st, const float* row_S, const float* gscale,
                                                     const float* inv_n, T* grad, int64_t ldg) {
  const int row = blockIdx.x;
  const float a = ms[row], ia = 1.f / ss[row], b = mt[row], ib = 1.f / st[row], S = row_S[row];
  const float c = gscale[0] * inv_n[0];
  const T* s = zs + (int64_t)row * lds;
  const T* t = zt + (int64_t)row * ldt;
  T* gr = grad + (int64_t)row * ldg;
  auto elem = [&](float zsv, float ztv) {
    const float ps = fast_expf(zsv - a) * ia, pt = fast_expf(ztv - b) * ib;
    const float d = ps - pt;
    const float sg = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
    return ps * (sg - S) * c;
  };
  int j0 = 0;
  if (al16p(s) && al16p(t) && al16p(gr)) {   // each thread reads its 16 bytes before writing them
    constexpr int VN = VN16<T>;
    const int nv = V / VN;
    for (int q = threadIdx.x; q < nv; q += 256) {
      float vs[VN], vt[VN];
      ld16(s + q * VN, vs);
      ld16(t + q * VN, vt);
#pragma unroll
      for (int e = 0; e < VN; ++e) vs[e] = elem(vs[e], vt[e]);
      st16(gr + q * VN, vs);
    }
    j0 = nv * VN;
  }
  for (int j = j0 + threadIdx.x; j < V; j += 256) Elem<T>::store(gr + j, elem(ldf(s + j), ldf(t + j)));
}

// Reverse KL forward: row_kl = sum ps * (ls - lt).
template <typename T>
__global__ __launch_bounds__(256) void kl_fwd_kernel(const T* __restrict__ zs, int64_t lds, const T* __restrict__ zt,
                                                     int64_t ldt, int V, const float* ms, const float* ss,
                                                     const float* mt, const float* st, float* row_kl) {
  __shared__ float red[32];
  const int row = blockIdx.x;
  const float la = ms[row] + logf(ss[row]), lb = mt[row] + logf(st[row]);
  const T* s = zs + (int64_t)row * lds;
  const T* t = zt + (int64_t)row * ldt;
  float kl = 0.f;
  auto elem = [&](float zsv, float ztv) {
    const float ls = zsv - la, lt = ztv - lb;
    kl += fast_expf(ls) * (ls - lt);
  };
  int j0 = 0;
  if (al16p(s) && al16p(t)) {
    constexpr int VN = VN16<T>;
    const int nv = V / VN;
    for (int q = threadIdx.x; q < nv; q += 256) {
      float vs[VN], vt[VN];
      ld16(s + q * VN, vs);
      ld16(t + q * VN, vt);
#pragma unroll
      for (int e = 0; e < VN; ++e) elem(vs[e], vt[e]);
    }
    j0 = nv * VN;
  }
  for (int j = j0 + threadIdx.x; j < V; j += 256) elem(ldf(s + j), ldf(t + j));
  kl = block_sum(kl, red);
  if (threadIdx.x == 0) row_kl[row] = kl;
}

// Reverse KL backward: grad[j] = ps_j * ((ls_j - lt_j) - row_kl) * g * inv_n; grad may alias zs.
template <typename T>
__global__ __launch_bounds__(256) void kl_bwd_kernel(const T* zs, int64_t lds, const T* __restrict__ zt, int64_t ldt,
                                                     int V, const float* ms, const float* ss, const float* mt,
                                                     const float* st, const float* row_kl, const float* gscale,
                                                     const float* inv_n, T* grad, int64_t ldg) {
  const int row = blockIdx.x;
  const float la = ms[row] + logf(ss[row]), lb = mt[row] + logf(st[row]), k = row_kl[row];
  const float c = gscale[0] * inv_n[0];
  const T* s = zs + (int64_t)row * lds;
  const T* t = zt + (int64_t)row * ldt;
  T* gr = grad + (int64_t)row * ldg;
  auto elem = [&](float zsv, float ztv) {
    const float ls = zsv - la, lt = ztv - lb;
    return fast_expf(ls) * ((ls - lt) - k) * c;
  };
  int j0 = 0;
  if (al16p(s) && al16p(t) && al16p(gr)) {
    constexpr int VN = VN16<T>;
    const int nv = V / VN;
    for (int q = threadIdx.x; q < nv; q += 256) {
      float vs[VN], vt[VN];
      ld16(s + q * VN, vs);
      ld16(t + q * VN, vt);
#pragma unroll
      for (int e = 0; e < VN; ++e) vs[e] = elem(vs[e], vt[e]);
      st16(gr + q * VN, vs);
    }
    j0 = nv * VN;
  }
  for (int j = j0 + threadIdx.x; j < V; j += 256) Elem<T>::store(gr + j, elem(ldf(s + j), ldf(t + j)));
}

// out[0] = scale * inv_n * sum x (single workgroup, fixed summation order).
__global__ __launch_bounds__(1024) void sum_scaled_kernel(int64_t n, const float* __restrict__ x,
                                                          const float* inv_n, float* out) {
  __shared__ float red[32];
  float acc = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) acc += x[i];
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) out[0] = acc * (inv_n ? inv_n[0] : 1.f);
}

// ---------------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------------
#define DISPATCH_T(dtype, ...)                                       \
  do {                                                               \
    if ((dtype) == UNOK_BF16) { using T = bf16_t; __VA_ARGS__; }     \
    else if ((dtype) == UNOK_F32) { using T = float; __VA_ARGS__; }  \
    else return unok::set_error(UNOK_EINVAL, "bad dtype %d", (dtype)); \
  } while (0)

UNOK_EXPORT int unok_row_lse_update(int dtype, int R, int Vc, const void* z, int64_t ldz, int c0, const int64_t* tgt,
                                    float* run_max, float* run_sum, float* zt, int first, void* stream) {
  UNOK_REQUIRE(R >= 0 && Vc >= 0 && (R <= 1 || ldz >= Vc), UNOK_EINVAL, "row_lse_update: R=%d Vc=%d ldz=%lld", R, Vc,
               (long long)ldz);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL(row_lse_update_kernel<T>, dim3(R), dim3(256), 0, st, (const T*)z, ldz, Vc, c0,
                                       tgt, run_max, run_sum, zt, first));
  return unok::check_launch("row_lse_update");
}

// Merges the per-128-column-block softmax statistics of unok_lmhead_ce_stats into one (max,
// sum-exp) per row; one workgroup per row, blocks merged in a fixed order.
__global__ __launch_bounds__(256) void ce_parts_reduce_kernel(int nparts, const float* __restrict__ pmax,
                                                              const float* __restrict__ psum, int64_t ldp,
                                                              float* run_max, float* run_sum) {
  __shared__ float red[32];
  const int row = blockIdx.x;
  const float* pm = pmax + (int64_t)row * ldp;
  const float* ps = psum + (int64_t)row * ldp;
  float m = -INFINITY;
  for (int b = threadIdx.x; b < nparts; b += 256) m = fmaxf(m, pm[b]);
  m = block_max(m, red);
  float s = 0.f;
  for (int b = threadIdx.x; b < nparts; b += 256) s += ps[b] > 0.f ? ps[b] * fast_expf(pm[b] - m) : 0.f;
  s = block_sum(s, red);
  if (threadIdx.x == 0) { run_max[row] = m; run_sum[row] = s; }
}

UNOK_EXPORT int unok_ce_parts_reduce(int R, int nparts, const float* pmax, const float* psum, int64_t ldp,
                                     float* run_max, float* run_sum, void* stream) {
  UNOK_REQUIRE(R >= 0 && nparts > 0 && ldp >= nparts, UNOK_EINVAL, "ce_parts_reduce: bad sizes");
  if (R == 0) return 0;
  hipLaunchKernelGGL(ce_parts_reduce_kernel, dim3(R), dim3(256), 0, (hipStream_t)stream, nparts, pmax, psum, ldp,
                     run_max, run_sum);
  return unok::check_launch("ce_parts_reduce");
}

UNOK_EXPORT int unok_row_argmax_update(int dtype, int R, int Vc, const void* z, int64_t ldz, int c0, float* best_val,
                                       int64_t* best_idx, int first, void* stream) {
  UNOK_REQUIRE(R >= 0 && Vc >= 0 && (R <= 1 || ldz >= Vc), UNOK_EINVAL, "row_argmax_update: R=%d Vc=%d ldz=%lld", R, Vc,
               (long long)ldz);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL(row_argmax_update_kernel<T>, dim3(R), dim3(256), 0, st, (const T*)z, ldz, Vc,
                                       c0, best_val, best_idx, first));
  return unok::check_launch("row_argmax_update");
}

UNOK_EXPORT int unok_ce_finish(int R, const float* run_max, const float* run_sum, const float* zt, const float* w,
                               const float* inv_n, float* lse, float* loss, void* stream) {
  UNOK_REQUIRE(R >= 0, UNOK_EINVAL, "ce_finish: R=%d", R);
  hipLaunchKernelGGL(ce_finish_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, R, run_max, run_sum, zt, w, inv_n,
                     lse, loss);
  return unok::check_launch("ce_finish");
}

UNOK_EXPORT int unok_ce_grad_chunk(int out_dtype, int R, int Vc, const float* z, int64_t ldz, int c0, const float* lse,
                                   const int64_t* tgt, const float* w, const float* gscale, const float* inv_n,
                                   void* dz, int64_t lddz, void* stream) {
  UNOK_REQUIRE(R >= 0 && Vc >= 0 && (R <= 1 || (ldz >= Vc && lddz >= Vc)), UNOK_EINVAL,
               "ce_grad_chunk: R=%d Vc=%d ldz=%lld lddz=%lld", R, Vc, (long long)ldz, (long long)lddz);
  UNOK_REQUIRE(out_dtype == UNOK_BF16 || out_dtype == UNOK_F32, UNOK_EINVAL, "ce_grad_chunk: bad dtype %d", out_dtype);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  if (out_dtype == UNOK_BF16)
    hipLaunchKernelGGL(ce_grad_chunk_kernel<bf16_t>, dim3(R), dim3(256), 0, st, z, ldz, Vc, c0, lse, tgt, w, gscale,
                       inv_n, (bf16_t*)dz, lddz);
  else
    hipLaunchKernelGGL(ce_grad_chunk_kernel<float>, dim3(R), dim3(256), 0, st, z, ldz, Vc, c0, lse, tgt, w, gscale,
                       inv_n, (float*)dz, lddz);
  return unok::check_launch("ce_grad_chunk");
}

UNOK_EXPORT int unok_softmax_stats(int dtype, int R, int V, const void* z, int64_t ldz, float* mx, float* se,
                                   void* stream) {
  UNOK_REQUIRE(R >= 0 && V >= 0 && (R <= 1 || ldz >= V), UNOK_EINVAL, "softmax_stats: R=%d V=%d ldz=%lld", R, V, (long long)ldz);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL(softmax_stats_kernel<T>, dim3(R), dim3(256), 0, st, (const T*)z, ldz, V, mx, se));
  return unok::check_launch("softmax_stats");
}

UNOK_EXPORT int unok_tv_fwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                            const float* ms, const float* ss, const float* mt, const float* st_, float* row_l1,
                            float* row_S, void* stream) {
  UNOK_REQUIRE(R >= 0 && V >= 0 && (R <= 1 || (lds >= V && ldt >= V)), UNOK_EINVAL, "tv_fwd: R=%d V=%d", R, V);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL(tv_fwd_kernel<T>, dim3(R), dim3(256), 0, st, (const T*)zs, lds, (const T*)zt,
                                       ldt, V, ms, ss, mt, st_, row_l1, row_S));
  return unok::check_launch("tv_fwd");
}

UNOK_EXPORT int unok_tv_bwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                            const float* ms, const float* ss, const float* mt, const float* st_, const float* row_S,
                            const float* gscale, const float* inv_n, void* grad, int64_t ldg, void* stream) {
  UNOK_REQUIRE(R >= 0 && V >= 0 && (R <= 1 || (lds >= V && ldt >= V && ldg >= V)), UNOK_EINVAL, "tv_bwd: R=%d V=%d", R, V);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL(tv_bwd_kernel<T>, dim3(R), dim3(256), 0, st, (const T*)zs, lds, (const T*)zt,
                                       ldt, V, ms, ss, mt, st_, row_S, gscale, inv_n, (T*)grad, ldg));
  return unok::check_launch("tv_bwd");
}

UNOK_EXPORT int unok_kl_fwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                            const float* ms, const float* ss, const float* mt, const float* st_, float* row_kl,
                            void* stream) {
  UNOK_REQUIRE(R >= 0 && V >= 0 && (R <= 1 || (lds >= V && ldt >= V)), UNOK_EINVAL, "kl_fwd: R=%d V=%d", R, V);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL(kl_fwd_kernel<T>, dim3(R), dim3(256), 0, st, (const T*)zs, lds, (const T*)zt,
                                       ldt, V, ms, ss, mt, st_, row_kl));
  return unok::check_launch("kl_fwd");
}

UNOK_EXPORT int unok_kl_bwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                            const float* ms, const float* ss, const float* mt, const float* st_, const float* row_kl,
                            const float* gscale, const float* inv_n, void* grad, int64_t ldg, void* stream) {
  UNOK_REQUIRE(R >= 0 && V >= 0 && (R <= 1 || (lds >= V && ldt >= V && ldg >= V)), UNOK_EINVAL, "kl_bwd: R=%d V=%d", R, V);
  if (R == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL(kl_bwd_kernel<T>, dim3(R), dim3(256), 0, st, (const T*)zs, lds, (const T*)zt,
                                       ldt, V, ms, ss, mt, st_, row_kl, gscale, inv_n, (T*)grad, ldg));
  return unok::check_launch("kl_bwd");
}

UNOK_EXPORT int unok_sum_scaled(int64_t n, const float* x, const float* inv_n, float* out, void* stream) {
  UNOK_REQUIRE(n >= 0, UNOK_EINVAL, "sum_scaled: n=%lld", (long long)n);
  hipLaunchKernelGGL(sum_scaled_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, n, x, inv_n, out);
  return unok::check_launch("sum_scaled");
}
