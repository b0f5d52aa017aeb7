// Row-wise HBM-bound kernels of the Qwen3 decoder layer: RMSNorm, per-head q/k RMSNorm fused
// with rotary embedding, SwiGLU, embedding gather and index-mapped row copies.
//
// Semantics follow transformers' Qwen3 modules (modeling_qwen3.py): RMSNorm statistics in
// fp32, normalised value rounded to the storage type, then scaled by the weight; q/k norms are
// per 128-wide head before RoPE (rotate_half convention, angle = fl32(pos * inv_freq[i]));
// SwiGLU is down(silu(gate) * up). Every kernel reads and writes with 16-byte vectors and
// reduces with 64-lane wavefront shuffles.
#include "common.h"

template <typename T> struct Vec { static constexpr int N = 16 / sizeof(T); };

template <typename T>
__device__ __forceinline__ void load_vec(const T* p, float* out) {
  uint4 u = *(const uint4*)p;
  if constexpr (sizeof(T) == 2) {
    const bf16_t* h = (const bf16_t*)&u;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = bf16_to_f32(h[e]);
  } else {
    const float* f = (const float*)&u;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = f[e];
  }
}

template <typename T>
__device__ __forceinline__ void store_vec(T* p, const float* in) {
  uint4 u;
  if constexpr (sizeof(T) == 2) {
    u = make_uint4(pack2_bf16(in[0], in[1]), pack2_bf16(in[2], in[3]), pack2_bf16(in[4], in[5]),
                   pack2_bf16(in[6], in[7]));
  } else {
    float* f = (float*)&u;
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = in[e];
  }
  *(uint4*)p = u;
}

// ---------------------------------------------------------------------------------------
// RMSNorm: y = w * round(x * rstd), rstd = rsqrt(mean(x^2) + eps); one 256-thread block/row.
// ---------------------------------------------------------------------------------------
template <typename T, int MAXV>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const T* __restrict__ x, int64_t ldx, const T* __restrict__ w,
                                                          T* __restrict__ y, int64_t ldy, float* __restrict__ rstd,
                                                          int H, float eps) {
  constexpr int V = Vec<T>::N;
  __shared__ float red[32];
  const int row = blockIdx.x, nv = H / V;
  const T* xr = x + (int64_t)row * ldx;
  float v[MAXV][V];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < nv) {
      load_vec(xr + c * V, v[i]);
#pragma unroll
      for (int e = 0; e < V; ++e) ss += v[i][e] * v[i][e];
    }
  }
  ss = block_sum(ss, red);
  const float r = rsqrtf(ss / (float)H + eps);
  if (threadIdx.x == 0 && rstd) rstd[row] = r;
  T* yr = y + (int64_t)row * ldy;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < nv) {
      float wv[V], o[V];
      load_vec(w + c * V, wv);
#pragma unroll
      for (int e = 0; e < V; ++e) o[e] = Elem<T>::round(v[i][e] * r) * wv[e];
      store_vec(yr + c * V, o);
    }
  }
}

// dx = rstd * (g - xhat * mean(g * xhat)) + dres, g = dy * w, xhat = x * rstd.
template <typename T, int MAXV>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                                                          const T* __restrict__ w, const float* __restrict__ rstd,
                                                          const T* dres, T* dx, int H) {
  constexpr int V = Vec<T>::N;
  __shared__ float red[32];
  const int row = blockIdx.x, nv = H / V;
  const int64_t off = (int64_t)row * H;
  const float r = rstd[row];
  float g[MAXV][V], xh[MAXV][V];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < nv) {
      float dv[V], wv[V];
      load_vec(dy + off + c * V, dv);
      load_vec(x + off + c * V, xh[i]);
      load_vec(w + c * V, wv);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        xh[i][e] *= r;
        g[i][e] = dv[e] * wv[e];
        dot += g[i][e] * xh[i][e];
      }
    }
  }
  dot = block_sum(dot, red) / (float)H;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < nv) {
      float o[V];
      float rv[V];
      if (dres) load_vec(dres + off + c * V, rv);
#pragma unroll
      for (int e = 0; e < V; ++e) o[e] = r * (g[i][e] - xh[i][e] * dot) + (dres ? rv[e] : 0.f);
      store_vec(dx + off + c * V, o);
    }
  }
}

// ---------------------------------------------------------------------------------------
// q/k RMSNorm (optional) + RoPE. One wavefront per (row, head); lane i handles the RoPE pair
// (i, i + d/2). Reads the fused qkv projection output, writes contiguous q and k.
// ---------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void qknorm_rope_fwd_kernel(const T* __restrict__ qkv, int64_t ld, const T* wq,
                                                              const T* wk, const int64_t* __restrict__ pos,
                                                              const float* __restrict__ inv_freq, T* __restrict__ qo,
                                                              T* __restrict__ ko, float* __restrict__ rstd, int M,
                                                              int nq, int nk, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nh = nq + nk;
  if (item >= (int64_t)M * nh) return;
  const int row = (int)(item / nh), hd = (int)(item % nh);
  const bool isq = hd < nq;
  const T* src = qkv + (int64_t)row * ld + (int64_t)hd * d;
  T* dst = isq ? qo + ((int64_t)row * nq + hd) * d : ko + ((int64_t)row * nk + (hd - nq)) * d;
  const T* w = isq ? wq : wk;
  const int half = d >> 1;
  float x0[2], x1[2];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int i = lane + 64 * t;
    x0[t] = x1[t] = 0.f;
    if (i < half) {
      x0[t] = Elem<T>::load(src + i);
      x1[t] = Elem<T>::load(src + i + half);
      ss += x0[t] * x0[t] + x1[t] * x1[t];
    }
  }
  float r = 1.f;
  if (w) {
    ss = wave_sum(ss);
    r = rsqrtf(ss / (float)d + eps);
    if (lane == 0) rstd[(int64_t)row * nh + hd] = r;
  }
  const float p = (float)pos[row];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int i = lane + 64 * t;
    if (i < half) {
      float n0 = x0[t], n1 = x1[t];
      if (w) {
        n0 = Elem<T>::round(Elem<T>::round(n0 * r) * Elem<T>::load(w + i));
        n1 = Elem<T>::round(Elem<T>::round(n1 * r) * Elem<T>::load(w + i + half));
      }
      float s, c;
      sincosf(p * inv_freq[i], &s, &c);
      Elem<T>::store(dst + i, n0 * c - n1 * s);
      Elem<T>::store(dst + i + half, n1 * c + n0 * s);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void qknorm_rope_bwd_kernel(const T* __restrict__ dq, const T* __restrict__ dk,
                                                              const T* __restrict__ qkv, int64_t ld, const T* wq,
                                                              const T* wk, const int64_t* __restrict__ pos,
                                                              const float* __restrict__ inv_freq,
                                                              const float* __restrict__ rstd, T* __restrict__ dqkv,
                                                              int64_t ldd, int M, int nq, int nk, int d) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nh = nq + nk;
  if (item >= (int64_t)M * nh) return;
  const int row = (int)(item / nh), hd = (int)(item % nh);
  const bool isq = hd < nq;
  const T* dy = isq ? dq + ((int64_t)row * nq + hd) * d : dk + ((int64_t)row * nk + (hd - nq)) * d;
  const T* src = qkv + (int64_t)row * ld + (int64_t)hd * d;
  T* out = dqkv + (int64_t)row * ldd + (int64_t)hd * d;
  const T* w = isq ? wq : wk;
  const int half = d >> 1;
  const float p = (float)pos[row];
  const float r = w ? rstd[(int64_t)row * nh + hd] : 1.f;
  float g0[2], g1[2], xh0[2], xh1[2];
  float dot = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int i = lane + 64 * t;
    g0[t] = g1[t] = xh0[t] = xh1[t] = 0.f;
    if (i < half) {
      const float dy0 = Elem<T>::load(dy + i), dy1 = Elem<T>::load(dy + i + half);
      float s, c;
      sincosf(p * inv_freq[i], &s, &c);
      const float dn0 = dy0 * c + dy1 * s;
      const float dn1 = dy1 * c - dy0 * s;
      if (w) {
        xh0[t] = Elem<T>::load(src + i) * r;
        xh1[t] = Elem<T>::load(src + i + half) * r;
        g0[t] = dn0 * Elem<T>::load(w + i);
        g1[t] = dn1 * Elem<T>::load(w + i + half);
        dot += g0[t] * xh0[t] + g1[t] * xh1[t];
      } else {
        g0[t] = dn0;
        g1[t] = dn1;
      }
    }
  }
  if (w) dot = wave_sum(dot) / (float)d;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int i = lane + 64 * t;
    if (i < half) {
      if (w) {
        Elem<T>::store(out + i, r * (g0[t] - xh0[t] * dot));
        Elem<T>::store(out + i + half, r * (g1[t] - xh1[t] * dot));
      } else {
        Elem<T>::store(out + i, g0[t]);
        Elem<T>::store(out + i + half, g1[t]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// SwiGLU on the fused gate|up projection: out = round(silu(g)) * u.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float sigmoidf_(float g) { return 1.f / (1.f + expf(-g)); }

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const T* __restrict__ gu, int64_t ld, T* __restrict__ out,
                                                         int M, int F) {
  constexpr int V = Vec<T>::N;
  const int nv = F / V;
  const int64_t total = (int64_t)M * nv;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / nv, c = (i % nv) * V;
    float g[V], u[V], o[V];
    load_vec(gu + row * ld + c, g);
    load_vec(gu + row * ld + F + c, u);
#pragma unroll
    for (int e = 0; e < V; ++e) o[e] = Elem<T>::round(g[e] * sigmoidf_(g[e])) * u[e];
    store_vec(out + row * F + c, o);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ dout, const T* __restrict__ gu,
                                                         int64_t ld, T* __restrict__ dgu, int64_t ldd, int M, int F) {
  constexpr int V = Vec<T>::N;
  const int nv = F / V;
  const int64_t total = (int64_t)M * nv;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / nv, c = (i % nv) * V;
    float g[V], u[V], d[V], dg[V], du[V];
    load_vec(gu + row * ld + c, g);
    load_vec(gu + row * ld + F + c, u);
    load_vec(dout + row * F + c, d);
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float sg = sigmoidf_(g[e]);
      const float silu = Elem<T>::round(g[e] * sg);
      du[e] = d[e] * silu;
      dg[e] = d[e] * u[e] * sg * (1.f + g[e] * (1.f - sg));
    }
    store_vec(dgu + row * ldd + c, dg);
    store_vec(dgu + row * ldd + F + c, du);
  }
}

// ---------------------------------------------------------------------------------------
// Row gathers: embedding lookup and index-mapped row copies (16-byte vectors).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embedding_kernel(const int64_t* __restrict__ ids, const uint4* __restrict__ table,
                                                        uint4* __restrict__ out, int M, int nvec, int64_t vocab) {
  const int64_t total = (int64_t)M * nvec;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / nvec, c = i % nvec;
    int64_t id = ids[r];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // ids are validated on the host
    out[i] = table[id * nvec + c];
  }
}

// dst[dmap ? dmap[r] : r] = src[smap ? smap[r] : r] for r < M; row width in 16-byte vectors.
__global__ __launch_bounds__(256) void rows_copy_kernel(const uint4* __restrict__ src, int64_t lds,
                                                        const int32_t* __restrict__ smap, uint4* __restrict__ dst,
                                                        int64_t ldd, const int32_t* __restrict__ dmap, int M,
                                                        int nvec) {
  const int64_t total = (int64_t)M * nvec;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / nvec, c = i % nvec;
    const int64_t rs = smap ? smap[r] : r, rd = dmap ? dmap[r] : r;
    dst[rd * ldd + c] = src[rs * lds + c];
  }
}

// ---------------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------------
static int grid_for(int64_t work) {
  int64_t b = (work + 255) / 256;
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

#define DISPATCH_T(dtype, ...)                                       \
  do {                                                               \
    if ((dtype) == UNOK_BF16) { using T = bf16_t; __VA_ARGS__; }     \
    else if ((dtype) == UNOK_F32) { using T = float; __VA_ARGS__; }  \
    else return unok::set_error(UNOK_EINVAL, "bad dtype %d", (dtype)); \
  } while (0)

template <typename T>
static int rmsnorm_fwd_t(int M, int H, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, float* rstd,
                         float eps, hipStream_t st) {
  constexpr int V = Vec<T>::N;
  const int nv = H / V;
  const int maxv = (nv + 255) / 256;
  const T* X = (const T*)x; const T* W = (const T*)w; T* Y = (T*)y;
  if (maxv <= 1) hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, 1>), dim3(M), dim3(256), 0, st, X, ldx, W, Y, ldy, rstd, H, eps);
  else if (maxv <= 2) hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, 2>), dim3(M), dim3(256), 0, st, X, ldx, W, Y, ldy, rstd, H, eps);
  else if (maxv <= 4) hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, 4>), dim3(M), dim3(256), 0, st, X, ldx, W, Y, ldy, rstd, H, eps);
  else if (maxv <= 8) hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, 8>), dim3(M), dim3(256), 0, st, X, ldx, W, Y, ldy, rstd, H, eps);
  else return unok::set_error(UNOK_EUNSUPPORTED, "rmsnorm: hidden size %d too large", H);
  return unok::check_launch("rmsnorm_fwd");
}

UNOK_EXPORT int unok_rmsnorm_fwd(int dtype, int M, int H, const void* x, int64_t ldx, const void* w, void* y,
                                 int64_t ldy, float* rstd, float eps, void* stream) {
  if (M == 0) return 0;
  const int V = dtype == UNOK_BF16 ? 8 : 4;
  UNOK_REQUIRE(H > 0 && H % V == 0 && ldx % V == 0 && ldy % V == 0, UNOK_EALIGN,
               "rmsnorm_fwd: H=%d and strides must be multiples of %d", H, V);
  DISPATCH_T(dtype, return rmsnorm_fwd_t<T>(M, H, x, ldx, w, y, ldy, rstd, eps, (hipStream_t)stream));
}

template <typename T>
static int rmsnorm_bwd_t(int M, int H, const void* dy, const void* x, const void* w, const float* rstd,
                         const void* dres, void* dx, hipStream_t st) {
  constexpr int V = Vec<T>::N;
  const int maxv = (H / V + 255) / 256;
  const T* DY = (const T*)dy; const T* X = (const T*)x; const T* W = (const T*)w; const T* DR = (const T*)dres;
  T* DX = (T*)dx;
  if (maxv <= 1) hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, 1>), dim3(M), dim3(256), 0, st, DY, X, W, rstd, DR, DX, H);
  else if (maxv <= 2) hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, 2>), dim3(M), dim3(256), 0, st, DY, X, W, rstd, DR, DX, H);
  else if (maxv <= 4) hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, 4>), dim3(M), dim3(256), 0, st, DY, X, W, rstd, DR, DX, H);
  else if (maxv <= 8) hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, 8>), dim3(M), dim3(256), 0, st, DY, X, W, rstd, DR, DX, H);
  else return unok::set_error(UNOK_EUNSUPPORTED, "rmsnorm: hidden size %d too large", H);
  return unok::check_launch("rmsnorm_bwd");
}

// dx may alias dres (in-place accumulation of the residual-stream gradient).
UNOK_EXPORT int unok_rmsnorm_bwd(int dtype, int M, int H, const void* dy, const void* x, const void* w,
                                 const float* rstd, const void* dres, void* dx, void* stream) {
  if (M == 0) return 0;
  const int V = dtype == UNOK_BF16 ? 8 : 4;
  UNOK_REQUIRE(H > 0 && H % V == 0, UNOK_EALIGN, "rmsnorm_bwd: H=%d must be a multiple of %d", H, V);
  DISPATCH_T(dtype, return rmsnorm_bwd_t<T>(M, H, dy, x, w, rstd, dres, dx, (hipStream_t)stream));
}

UNOK_EXPORT int unok_qknorm_rope_fwd(int dtype, int M, int nq, int nk, int d, const void* qkv, int64_t ld,
                                     const void* wq, const void* wk, const int64_t* pos, const float* inv_freq,
                                     float eps, void* q_out, void* k_out, float* rstd, void* stream) {
  if (M == 0) return 0;
  UNOK_REQUIRE(d % 2 == 0 && d <= 256 && nq > 0 && nk >= 0, UNOK_EINVAL, "qknorm_rope: bad head geometry d=%d", d);
  UNOK_REQUIRE((wq == nullptr) == (wk == nullptr), UNOK_EINVAL, "qknorm_rope: q and k norms must both be given");
  const int64_t items = (int64_t)M * (nq + nk);
  const int blocks = (int)((items + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL((qknorm_rope_fwd_kernel<T>), dim3(blocks), dim3(256), 0, st, (const T*)qkv, ld,
                                       (const T*)wq, (const T*)wk, pos, inv_freq, (T*)q_out, (T*)k_out, rstd, M, nq,
                                       nk, d, eps));
  return unok::check_launch("qknorm_rope_fwd");
}

UNOK_EXPORT int unok_qknorm_rope_bwd(int dtype, int M, int nq, int nk, int d, const void* dq, const void* dk,
                                     const void* qkv, int64_t ld, const void* wq, const void* wk, const int64_t* pos,
                                     const float* inv_freq, const float* rstd, void* dqkv, int64_t ldd,
                                     void* stream) {
  if (M == 0) return 0;
  UNOK_REQUIRE(d % 2 == 0 && d <= 256, UNOK_EINVAL, "qknorm_rope_bwd: bad head dim %d", d);
  const int64_t items = (int64_t)M * (nq + nk);
  const int blocks = (int)((items + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL((qknorm_rope_bwd_kernel<T>), dim3(blocks), dim3(256), 0, st, (const T*)dq,
                                       (const T*)dk, (const T*)qkv, ld, (const T*)wq, (const T*)wk, pos, inv_freq, rstd,
                                       (T*)dqkv, ldd, M, nq, nk, d));
  return unok::check_launch("qknorm_rope_bwd");
}

UNOK_EXPORT int unok_swiglu_fwd(int dtype, int M, int F, const void* gu, int64_t ld, void* out, void* stream) {
  if (M == 0) return 0;
  const int V = dtype == UNOK_BF16 ? 8 : 4;
  UNOK_REQUIRE(F % V == 0 && ld % V == 0, UNOK_EALIGN, "swiglu: F=%d must be a multiple of %d", F, V);
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL((swiglu_fwd_kernel<T>), dim3(grid_for((int64_t)M * F / V)), dim3(256), 0, st,
                                       (const T*)gu, ld, (T*)out, M, F));
  return unok::check_launch("swiglu_fwd");
}

UNOK_EXPORT int unok_swiglu_bwd(int dtype, int M, int F, const void* dout, const void* gu, int64_t ld, void* dgu,
                                int64_t ldd, void* stream) {
  if (M == 0) return 0;
  const int V = dtype == UNOK_BF16 ? 8 : 4;
  UNOK_REQUIRE(F % V == 0 && ld % V == 0 && ldd % V == 0, UNOK_EALIGN, "swiglu_bwd: F=%d must be a multiple of %d", F, V);
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_T(dtype, hipLaunchKernelGGL((swiglu_bwd_kernel<T>), dim3(grid_for((int64_t)M * F / V)), dim3(256), 0, st,
                                       (const T*)dout, (const T*)gu, ld, (T*)dgu, ldd, M, F));
  return unok::check_launch("swiglu_bwd");
}

UNOK_EXPORT int unok_embedding(int elem_bytes, int M, int H, const int64_t* ids, const void* table, int64_t vocab,
                               void* out, void* stream) {
  if (M == 0) return 0;
  UNOK_REQUIRE(((int64_t)H * elem_bytes) % 16 == 0, UNOK_EALIGN, "embedding: row bytes must be a multiple of 16");
  const int nvec = (int)((int64_t)H * elem_bytes / 16);
  hipLaunchKernelGGL(embedding_kernel, dim3(grid_for((int64_t)M * nvec)), dim3(256), 0, (hipStream_t)stream, ids,
                     (const uint4*)table, (uint4*)out, M, nvec, vocab);
  return unok::check_launch("embedding");
}

UNOK_EXPORT int unok_rows_copy(int row_bytes, int M, const void* src, int64_t ld_src_bytes, const int32_t* smap,
                               void* dst, int64_t ld_dst_bytes, const int32_t* dmap, void* stream) {
  if (M == 0) return 0;
  UNOK_REQUIRE(row_bytes % 16 == 0 && ld_src_bytes % 16 == 0 && ld_dst_bytes % 16 == 0, UNOK_EALIGN,
               "rows_copy: row bytes and strides must be multiples of 16");
  const int nvec = row_bytes / 16;
  hipLaunchKernelGGL(rows_copy_kernel, dim3(grid_for((int64_t)M * nvec)), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)src, ld_src_bytes / 16, smap, (uint4*)dst, ld_dst_bytes / 16, dmap, M, nvec);
  return unok::check_launch("rows_copy");
}
