// Row-wise HBM-bound kernels of the Qwen3 decoder layer: RMSNorm, per-head q/k RMSNorm fused
// with rotary embedding, SwiGLU, embedding gather and index-mapped row copies.
//
// Semantics follow transformers' Qwen3 modules (modeling_qwen3.py): RMSNorm statistics in
// fp32; q/k norms are per 128-wide head before RoPE (rotate_half convention, angle =
// fl32(pos * inv_freq[i])); SwiGLU is down(silu(gate) * up). Each kernel keeps its whole
// computation in fp32 and rounds once, at the store (normalised value times weight, then the
// rotation; silu(gate) times up), where a bf16 module rounds after every operation: the step's
// LoRA gradients stay closer to the fp32 computation. Every kernel reads and writes with 16-byte
// vectors and reduces with 64-lane wavefront shuffles.
#include "common.h"

#include <type_traits>

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
// RMSNorm: y = w * x * rstd, rstd = rsqrt(mean(x^2) + eps), in fp32 and rounded once at the store;
// one 256-thread block/row.
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
      for (int e = 0; e < V; ++e) o[e] = v[i][e] * r * wv[e];
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
// q/k RMSNorm (optional) + RoPE. One wavefront per row covers all q and k heads of the row,
// HPW heads per pass: each lane owns 16 contiguous bytes (EPL elements) of a head and the RoPE
// partner elements (i +- d/2) sit LPH/2 lanes away, fetched with a lane shuffle. The row's
// angles fl32(pos * inv_freq[j]) are evaluated once per row (one sincosf per lane) into LDS.
// Reads the fused qkv projection output, writes contiguous q and k.
// ---------------------------------------------------------------------------------------
// Head passes whose loads the qk-norm / RoPE kernels issue together.
constexpr int QKR_GROUP = 5;

template <typename T> struct Vec16;
template <> struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const uint4 u, float (&v)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = __uint_as_float(w[i] << 16); v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u); }
  }
  __device__ __forceinline__ static void load(const bf16_t* p, float (&v)[8]) { unpack(*(const uint4*)p, v); }
  __device__ __forceinline__ static void store(bf16_t* p, const float (&v)[8]) {
    *(uint4*)p = make_uint4(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]), pack2_bf16(v[4], v[5]), pack2_bf16(v[6], v[7]));
  }
};
template <> struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(const uint4 u, float (&v)[4]) {
    v[0] = __uint_as_float(u.x); v[1] = __uint_as_float(u.y); v[2] = __uint_as_float(u.z); v[3] = __uint_as_float(u.w);
  }
  __device__ __forceinline__ static void load(const float* p, float (&v)[4]) { unpack(*(const uint4*)p, v); }
  __device__ __forceinline__ static void store(float* p, const float (&v)[4]) { *(float4*)p = make_float4(v[0], v[1], v[2], v[3]); }
};

// Angles of one row into LDS (cs, sn: d/2 floats each, one wavefront).
__device__ __forceinline__ void rope_angles(float p, const float* __restrict__ inv_freq, int half, float* cs,
                                            float* sn, int lane) {
  for (int j = lane; j < half; j += 64) {
    float sv, cv;
    sincosf(p * inv_freq[j], &sv, &cv);
    cs[j] = cv;
    sn[j] = sv;
  }
}

// N elements of T at p as floats, and back (N * sizeof(T) is 8 or 16 bytes, aligned).
template <typename T, int N> __device__ __forceinline__ void ld_elems(const T* p, float (&v)[N]) {
  if constexpr (std::is_same<T, float>::value) {
    static_assert(N == 4, "fp32 groups of 4");
    const float4 f = *(const float4*)p;
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else if constexpr (N == 8) {
    Vec16<bf16_t>::load(p, v);
  } else {
    static_assert(N == 4, "bf16 groups of 4 or 8");
    const uint2 u = *(const uint2*)p;
    v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xffff0000u);
  }
}
template <typename T, int N> __device__ __forceinline__ void st_elems(T* p, const float (&v)[N]) {
  if constexpr (std::is_same<T, float>::value) {
    static_assert(N == 4, "fp32 groups of 4");
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (N == 8) {
    Vec16<bf16_t>::store(p, v);
  } else {
    static_assert(N == 4, "bf16 groups of 4 or 8");
    *(uint2*)p = make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
  }
}

// TI: element type of the qkv input (the projection output; fp32 for bf16 models keeps the q/k
// values unrounded up to the normalisation); TO: element type of q, k, the norm weights and the
// optional copy of the v heads into vo [M, nk*D] (row stride ldv), which the attention kernels
// read as their V operand.
template <typename TI, typename TO, int D>
__global__ __launch_bounds__(256) void qknorm_rope_fwd_kernel(const TI* __restrict__ qkv, int64_t ld, const TO* wq,
                                                              const TO* wk, const int64_t* __restrict__ pos,
                                                              const float* __restrict__ inv_freq, TO* __restrict__ qo,
                                                              TO* __restrict__ ko, TO* __restrict__ vo, int64_t ldv,
                                                              float* __restrict__ rstd, int M, int nq, int nk,
                                                              float eps) {
  constexpr int EPL = Vec16<TI>::N, LPH = D / EPL, HPW = 64 / LPH, HALF = D / 2;
  static_assert(LPH >= 2 && LPH <= 64 && 64 % LPH == 0, "head geometry");
  __shared__ float s_cs[4][HALF], s_sn[4][HALF];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + w;
  if (row < M) rope_angles((float)pos[row], inv_freq, HALF, s_cs[w], s_sn[w], lane);
  __syncthreads();
  if (row >= M) return;
  const int hh = lane / LPH, c0 = (lane % LPH) * EPL;
  const int j0 = c0 % HALF;
  const float sgn = c0 < HALF ? -1.f : 1.f;
  float cv[EPL], sv[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) { cv[e] = s_cs[w][j0 + e]; sv[e] = s_sn[w][j0 + e]; }
  const int nh = nq + nk;
  const int nall = vo != nullptr ? nh + nk : nh;   // v heads follow the k heads in qkv
  const bool norm = wq != nullptr;
  float wqv[EPL], wkv[EPL];
  if (norm) {
    ld_elems<TO, EPL>(wq + c0, wqv);
    ld_elems<TO, EPL>(wk + c0, wkv);
  }
  // Heads in groups of QKR_GROUP passes: the group's loads are all issued before its arithmetic,
  // so each wavefront keeps several KB of the row in flight instead of one pass's 1 KB.
  for (int hb0 = 0; hb0 < nall; hb0 += HPW * QKR_GROUP) {
    uint4 raw[QKR_GROUP];
#pragma unroll
    for (int gi = 0; gi < QKR_GROUP; ++gi) {
      const int head = hb0 + gi * HPW + hh;
      raw[gi] = head < nall ? *(const uint4*)(qkv + (int64_t)row * ld + (int64_t)head * D + c0) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int gi = 0; gi < QKR_GROUP; ++gi) {
      const int head = hb0 + gi * HPW + hh;
      const bool valid = head < nh;
      const bool isq = head < nq;
      float x[EPL];
      Vec16<TI>::unpack(raw[gi], x);
      if (head >= nh) {      // a v head (or past the row): copied, no norm or rotation
        if (head < nall) st_elems<TO, EPL>(vo + (int64_t)row * ldv + (int64_t)(head - nh) * D + c0, x);
        continue;
      }
      if (norm) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) ss += x[e] * x[e];
#pragma unroll
        for (int o = LPH / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        const float r = rsqrtf(ss / (float)D + eps);
        if (valid && lane % LPH == 0) rstd[(int64_t)row * nh + head] = r;
#pragma unroll
        for (int e = 0; e < EPL; ++e)
          x[e] = valid ? x[e] * r * (isq ? wqv[e] : wkv[e]) : 0.f;
      }
      float out[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float y = __shfl_xor(x[e], LPH / 2, 64);   // partner element i +- d/2
        out[e] = x[e] * cv[e] + sgn * y * sv[e];
      }
      if (valid) {
        TO* dst = isq ? qo + ((int64_t)row * nq + head) * D : ko + ((int64_t)row * nk + (head - nq)) * D;
        st_elems<TO, EPL>(dst + c0, out);
      }
    }
  }
}

// TI: element type of dq and dk; TX: of the pre-norm input (the q/k columns of qkv, row stride
// ld); TO: of dqkv and the norm weights.
template <typename TI, typename TX, typename TO, int D>
__global__ __launch_bounds__(256) void qknorm_rope_bwd_kernel(const TI* __restrict__ dq, const TI* __restrict__ dk,
                                                              const TX* __restrict__ qkv, int64_t ld, const TO* wq,
                                                              const TO* wk, const int64_t* __restrict__ pos,
                                                              const float* __restrict__ inv_freq,
                                                              const float* __restrict__ rstd, TO* __restrict__ dqkv,
                                                              int64_t ldd, int M, int nq, int nk) {
  constexpr int EPL = Vec16<TI>::N, LPH = D / EPL, HPW = 64 / LPH, HALF = D / 2;
  static_assert(LPH >= 2 && LPH <= 64 && 64 % LPH == 0, "head geometry");
  __shared__ float s_cs[4][HALF], s_sn[4][HALF];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + w;
  if (row < M) rope_angles((float)pos[row], inv_freq, HALF, s_cs[w], s_sn[w], lane);
  __syncthreads();
  if (row >= M) return;
  const int hh = lane / LPH, c0 = (lane % LPH) * EPL;
  const int j0 = c0 % HALF;
  // inverse rotation: dn_i = dy_i c + dy_{i+h} s (first half), dn_i = dy_i c - dy_{i-h} s (second)
  const float sgn = c0 < HALF ? 1.f : -1.f;
  float cv[EPL], sv[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) { cv[e] = s_cs[w][j0 + e]; sv[e] = s_sn[w][j0 + e]; }
  const int nh = nq + nk;
  const bool norm = wq != nullptr;
  float wqv[EPL], wkv[EPL];
  if (norm) {
    ld_elems<TO, EPL>(wq + c0, wqv);
    ld_elems<TO, EPL>(wk + c0, wkv);
  }
  // As in the forward: each group's loads (upstream gradient, input row, rstd) go out before its
  // arithmetic.
  for (int hb0 = 0; hb0 < nh; hb0 += HPW * QKR_GROUP) {
    uint4 rdy[QKR_GROUP];
    float rx[QKR_GROUP][EPL];
    float rs[QKR_GROUP];
#pragma unroll
    for (int gi = 0; gi < QKR_GROUP; ++gi) {
      const int head = hb0 + gi * HPW + hh;
      const bool valid = head < nh;
      const bool isq = head < nq;
      rdy[gi] = valid ? *(const uint4*)(isq ? dq + ((int64_t)row * nq + head) * D + c0
                                            : dk + ((int64_t)row * nk + (head - nq)) * D + c0)
                      : make_uint4(0, 0, 0, 0);
      if (valid && norm) ld_elems<TX, EPL>(qkv + (int64_t)row * ld + (int64_t)head * D + c0, rx[gi]);
      else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) rx[gi][e] = 0.f;
      }
      rs[gi] = valid && norm ? rstd[(int64_t)row * nh + head] : 0.f;
    }
#pragma unroll
    for (int gi = 0; gi < QKR_GROUP; ++gi) {
      const int head = hb0 + gi * HPW + hh;
      const bool valid = head < nh;
      const bool isq = head < nq;
      float dy[EPL];
      Vec16<TI>::unpack(rdy[gi], dy);
      float g[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float y = __shfl_xor(dy[e], LPH / 2, 64);
        g[e] = dy[e] * cv[e] + sgn * y * sv[e];
      }
      if (norm) {
        const float r = rs[gi];
        float x[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) x[e] = rx[gi][e];
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          x[e] *= r;            // x-hat
          g[e] *= valid ? (isq ? wqv[e] : wkv[e]) : 0.f;
          dot += g[e] * x[e];
        }
#pragma unroll
        for (int o = LPH / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
        dot /= (float)D;
#pragma unroll
        for (int e = 0; e < EPL; ++e) g[e] = r * (g[e] - x[e] * dot);
      }
      if (valid) st_elems<TO, EPL>(dqkv + (int64_t)row * ldd + (int64_t)head * D + c0, g);
    }
  }
}

// ---------------------------------------------------------------------------------------
// SwiGLU on the fused gate|up projection: out = silu(g) * u in fp32, rounded once at the store.
// ---------------------------------------------------------------------------------------

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
    for (int e = 0; e < V; ++e) o[e] = g[e] * sigmoidf_(g[e]) * u[e];
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
      if constexpr (std::is_same<T, bf16_t>::value) {
        swiglu_grad(d[e], g[e], u[e], dg[e], du[e]);
      } else {
        const float sg = sigmoidf_(g[e]);
        du[e] = d[e] * (g[e] * sg);
        dg[e] = d[e] * u[e] * sg * (1.f + g[e] * (1.f - sg));
      }
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

// Input / output element-type pairs of the q/k-norm kernels: (fp32, fp32), (bf16, bf16) and
// (fp32 in, bf16 out).
#define QKR_DISPATCH(TO_CODE, TI_CODE, ...)                                                          \
  do {                                                                                              \
    if ((TO_CODE) == UNOK_F32 && (TI_CODE) == UNOK_F32) { using TO = float; using TI = float; __VA_ARGS__; }  \
    else if ((TO_CODE) == UNOK_BF16 && (TI_CODE) == UNOK_BF16) { using TO = bf16_t; using TI = bf16_t; __VA_ARGS__; } \
    else if ((TO_CODE) == UNOK_BF16 && (TI_CODE) == UNOK_F32) { using TO = bf16_t; using TI = float; __VA_ARGS__; } \
    else return unok::set_error(UNOK_EINVAL, "qknorm_rope: unsupported element types (out %d, in %d)", \
                                (int)(TO_CODE), (int)(TI_CODE));                                    \
  } while (0)

UNOK_EXPORT int unok_qknorm_rope_fwd(int dtype, int qkv_dtype, int M, int nq, int nk, int d, const void* qkv,
                                     int64_t ld, const void* wq, const void* wk, const int64_t* pos,
                                     const float* inv_freq, float eps, void* q_out, void* k_out, void* v_out,
                                     int64_t ldv, float* rstd, void* stream) {
  if (M == 0) return 0;
  UNOK_REQUIRE((d == 64 || d == 128) && nq > 0 && nk >= 0, UNOK_EINVAL, "qknorm_rope: head dim %d not in {64,128}", d);
  UNOK_REQUIRE((wq == nullptr) == (wk == nullptr), UNOK_EINVAL, "qknorm_rope: q and k norms must both be given");
  UNOK_REQUIRE(ld % 8 == 0 && ((uintptr_t)qkv & 15) == 0 && ((uintptr_t)q_out & 15) == 0 && ((uintptr_t)k_out & 15) == 0 &&
                   (v_out == nullptr || (ldv % 8 == 0 && ((uintptr_t)v_out & 15) == 0)),
               UNOK_EALIGN, "qknorm_rope: rows must be 16-byte aligned");
  const int blocks = (M + 3) / 4;
  hipStream_t st = (hipStream_t)stream;
  if (d == 128)
    QKR_DISPATCH(dtype, qkv_dtype, hipLaunchKernelGGL((qknorm_rope_fwd_kernel<TI, TO, 128>), dim3(blocks), dim3(256), 0,
                                                      st, (const TI*)qkv, ld, (const TO*)wq, (const TO*)wk, pos, inv_freq,
                                                      (TO*)q_out, (TO*)k_out, (TO*)v_out, ldv, rstd, M, nq, nk, eps));
  else
    QKR_DISPATCH(dtype, qkv_dtype, hipLaunchKernelGGL((qknorm_rope_fwd_kernel<TI, TO, 64>), dim3(blocks), dim3(256), 0,
                                                      st, (const TI*)qkv, ld, (const TO*)wq, (const TO*)wk, pos, inv_freq,
                                                      (TO*)q_out, (TO*)k_out, (TO*)v_out, ldv, rstd, M, nq, nk, eps));
  return unok::check_launch("qknorm_rope_fwd");
}

UNOK_EXPORT int unok_qknorm_rope_bwd(int dtype, int grad_dtype, int x_dtype, int M, int nq, int nk, int d,
                                     const void* dq, const void* dk, const void* qkv, int64_t ld, const void* wq,
                                     const void* wk, const int64_t* pos, const float* inv_freq, const float* rstd,
                                     void* dqkv, int64_t ldd, void* stream) {
  if (M == 0) return 0;
  UNOK_REQUIRE(d == 64 || d == 128, UNOK_EINVAL, "qknorm_rope_bwd: head dim %d not in {64,128}", d);
  UNOK_REQUIRE(ld % 8 == 0 && ldd % 8 == 0 && ((uintptr_t)qkv & 15) == 0 && ((uintptr_t)dqkv & 15) == 0 &&
                   ((uintptr_t)dq & 15) == 0 && ((uintptr_t)dk & 15) == 0,
               UNOK_EALIGN, "qknorm_rope_bwd: rows must be 16-byte aligned");
  const int blocks = (M + 3) / 4;
  hipStream_t st = (hipStream_t)stream;
#define QKR_BWD(TX_T)                                                                                          \
  do {                                                                                                         \
    if (d == 128)                                                                                              \
      hipLaunchKernelGGL((qknorm_rope_bwd_kernel<TI, TX_T, TO, 128>), dim3(blocks), dim3(256), 0, st, (const TI*)dq, \
                         (const TI*)dk, (const TX_T*)qkv, ld, (const TO*)wq, (const TO*)wk, pos, inv_freq, rstd,  \
                         (TO*)dqkv, ldd, M, nq, nk);                                                          \
    else                                                                                                       \
      hipLaunchKernelGGL((qknorm_rope_bwd_kernel<TI, TX_T, TO, 64>), dim3(blocks), dim3(256), 0, st, (const TI*)dq, \
                         (const TI*)dk, (const TX_T*)qkv, ld, (const TO*)wq, (const TO*)wk, pos, inv_freq, rstd,  \
                         (TO*)dqkv, ldd, M, nq, nk);                                                          \
  } while (0)
  // the pre-norm input is either of the gradient's type, or bf16 beside fp32 gradients
  UNOK_REQUIRE(x_dtype == grad_dtype || (x_dtype == UNOK_BF16 && grad_dtype == UNOK_F32 && dtype == UNOK_BF16),
               UNOK_EINVAL, "qknorm_rope_bwd: input type %d with gradient type %d", x_dtype, grad_dtype);
  if (x_dtype == grad_dtype)
    QKR_DISPATCH(dtype, grad_dtype, QKR_BWD(TI));
  else
    QKR_DISPATCH(dtype, grad_dtype, QKR_BWD(bf16_t));
#undef QKR_BWD
  return unok::check_launch("qknorm_rope_bwd");
}

// cos_tab / sin_tab [P, half]: cos and sin of fl32(p * inv_freq[j]), the angles unok_qknorm_rope_fwd
// evaluates per row, tabulated for the fused q|k|v projection epilogue.
__global__ __launch_bounds__(256) void rope_table_kernel(int P, int half, const float* __restrict__ inv_freq,
                                                         float* __restrict__ cs, float* __restrict__ sn) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)P * half) return;
  const int p = (int)(i / half), j = (int)(i % half);
  float sv, cv;
  sincosf((float)p * inv_freq[j], &sv, &cv);
  cs[i] = cv;
  sn[i] = sv;
}

UNOK_EXPORT int unok_rope_table(int P, int half, const float* inv_freq, float* cos_tab, float* sin_tab, void* stream) {
  UNOK_REQUIRE(P >= 0 && half > 0, UNOK_EINVAL, "rope_table: P=%d half=%d", P, half);
  if (P == 0) return 0;
  const int64_t n = (int64_t)P * half;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, P, half,
                     inv_freq, cos_tab, sin_tab);
  return unok::check_launch("rope_table");
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
