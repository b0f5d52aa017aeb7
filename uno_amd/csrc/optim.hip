// Optimizer kernels over the flat LoRA state (all lora_A/lora_B tensors live in one fp32
// buffer; master, gradient, exp_avg and exp_avg_sq are parallel buffers of the same layout).
//
// Step semantics follow training/train.py:282-288: global-norm gradient clipping to
// max_grad_norm = 1.0 (torch.nn.utils.clip_grad_norm_: coef = max_norm / (norm + 1e-6), clamped
// to 1, applied to every gradient), then torch.optim.AdamW (bias-corrected, decoupled weight
// decay p *= 1 - lr*wd, step_size = lr / (1 - b1^t), denom = sqrt(v) / sqrt(1 - b2^t) + eps).
// The same pass refreshes the bf16 compute copy used by the GEMM kernels (LoRA B scaled by
// alpha/r); transposed compute copies are produced by a batched tile-transpose.
#include "common.h"

// Partial sums of squares: 16-byte loads over the 4-aligned body (the flat buffers are
// 256-byte aligned), scalar loads for the tail; fixed order per workgroup.
__global__ __launch_bounds__(256) void sumsq_kernel(int64_t n, const float* __restrict__ x, float* __restrict__ part) {
  __shared__ float red[32];
  float s = 0.f;
  const int64_t n4 = ((uintptr_t)x & 15) == 0 ? n / 4 : 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
    const float4 v = ((const float4*)x)[i];
    s += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) s += x[i] * x[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

// out[0] = global norm, out[1] = clip coefficient.
__global__ __launch_bounds__(256) void clip_coef_kernel(int nparts, const float* __restrict__ part, float max_norm,
                                                        float* out) {
  __shared__ double red[256];
  double s = 0.0;
  for (int i = threadIdx.x; i < nparts; i += 256) s += (double)part[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float norm = (float)sqrt(red[0]);
    out[0] = norm;
    out[1] = max_norm > 0.f ? fminf(1.f, max_norm / (norm + 1e-6f)) : 1.f;
  }
}

struct AdamArgs {
  float* p; float* g; float* m; float* v;
  void* copy;              // compute copy (may be null), bf16 or fp32 per copy_f32
  int copy_f32;
  int64_t n, n_unscaled;   // elements [n_unscaled, n) are copied with copy_scale
  float copy_scale;
  const float* clip;       // device [norm, coef] (may be null)
  float lr, b1, b2, eps, wd, bc1, bc2_sqrt;
};

// One element's update (torch.optim.AdamW's arithmetic order); returns the new parameter.
__device__ __forceinline__ float adamw_one(const AdamArgs& a, float coef, float step_size, float& g, float p, float& m,
                                           float& v) {
  g *= coef;
  if (a.wd != 0.f) p *= 1.f - a.lr * a.wd;
  m = m + (1.f - a.b1) * (g - m);
  v = v * a.b2 + (1.f - a.b2) * g * g;
  const float denom = sqrtf(v) / a.bc2_sqrt + a.eps;
  return p - step_size * (m / denom);
}

// Four elements per thread with 16-byte loads and stores over the body (all flat buffers are
// 256-byte aligned; the body is used only when every pointer is), one element per thread for
// the tail. The bf16 compute copy is written 8 bytes at a time.
__global__ __launch_bounds__(256) void adamw_kernel(const AdamArgs a) {
  const float coef = a.clip ? a.clip[1] : 1.f;
  const float step_size = a.lr / a.bc1;
  const bool vec = (((uintptr_t)a.p | (uintptr_t)a.g | (uintptr_t)a.m | (uintptr_t)a.v) & 15) == 0 &&
                   ((uintptr_t)a.copy & (a.copy_f32 ? 15 : 7)) == 0 && (a.n_unscaled & 3) == 0;
  const int64_t n4 = vec ? a.n / 4 : 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
    float4 g = ((const float4*)a.g)[i], p = ((const float4*)a.p)[i];
    float4 m = ((const float4*)a.m)[i], v = ((const float4*)a.v)[i];
    p.x = adamw_one(a, coef, step_size, g.x, p.x, m.x, v.x);
    p.y = adamw_one(a, coef, step_size, g.y, p.y, m.y, v.y);
    p.z = adamw_one(a, coef, step_size, g.z, p.z, m.z, v.z);
    p.w = adamw_one(a, coef, step_size, g.w, p.w, m.w, v.w);
    ((float4*)a.p)[i] = p;
    ((float4*)a.m)[i] = m;
    ((float4*)a.v)[i] = v;
    ((float4*)a.g)[i] = g;
    if (a.copy) {
      const float sc = 4 * i < a.n_unscaled ? 1.f : a.copy_scale;
      if (a.copy_f32) {
        ((float4*)a.copy)[i] = make_float4(p.x * sc, p.y * sc, p.z * sc, p.w * sc);
      } else {
        ((uint2*)a.copy)[i] = make_uint2(pack2_bf16(p.x * sc, p.y * sc), pack2_bf16(p.z * sc, p.w * sc));
      }
    }
  }
  for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n; i += stride) {
    float g = a.g[i], m = a.m[i], v = a.v[i];
    const float p = adamw_one(a, coef, step_size, g, a.p[i], m, v);
    a.p[i] = p;
    a.m[i] = m;
    a.v[i] = v;
    a.g[i] = g;
    if (a.copy) {
      const float c = i < a.n_unscaled ? p : p * a.copy_scale;
      if (a.copy_f32) ((float*)a.copy)[i] = c;
      else ((bf16_t*)a.copy)[i] = f32_to_bf16(c);
    }
  }
}

// Refreshes the bf16 compute copy without an update (initialisation, after loading weights).
template <typename T>
__global__ __launch_bounds__(256) void cast_copy_kernel(int64_t n, int64_t n_unscaled, float scale,
                                                        const float* __restrict__ p, T* __restrict__ copy) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    Elem<T>::store(copy + i, i < n_unscaled ? p[i] : p[i] * scale);
}

// Batched transpose of bf16 matrices: job j = {src_off, rows, cols, dst_off, tile_begin, 0,0,0}
// (offsets in elements into the src/dst base buffers). One 64x64 tile per workgroup.
template <typename T>
__global__ __launch_bounds__(256) void transpose_jobs_kernel(const int64_t* __restrict__ jobs, int njobs,
                                                             const T* __restrict__ src, T* __restrict__ dst) {
  __shared__ T tile[64][65];
  const int64_t bid = blockIdx.x;
  int lo = 0, hi = njobs - 1;
  while (lo < hi) {  // last job with tile_begin <= bid
    const int mid = (lo + hi + 1) >> 1;
    if (jobs[mid * 8 + 4] <= bid) lo = mid; else hi = mid - 1;
  }
  const int64_t* j = jobs + lo * 8;
  const int64_t rows = j[1], cols = j[2];
  const int64_t t = bid - j[4];
  const int64_t tcols = (cols + 63) / 64;
  const int64_t r0 = (t / tcols) * 64, c0 = (t % tcols) * 64;
  const T* s = src + j[0];
  T* d = dst + j[3];
  if constexpr (sizeof(T) == 2) {
    // bf16 matrices whose sides are multiples of 8 (and 16-byte aligned): 16-byte loads of 8
    // source columns and 16-byte stores of 8 destination columns, the tile transposed in LDS.
    if (rows % 8 == 0 && cols % 8 == 0 && (((uintptr_t)s | (uintptr_t)d) & 15) == 0) {
      __shared__ __attribute__((aligned(16))) T tv[64][72];
      for (int e = threadIdx.x; e < 64 * 8; e += 256) {
        const int rr = e / 8, cc = (e % 8) * 8;
        const int64_t r = r0 + rr, c = c0 + cc;
        if (r < rows && c < cols) *(uint4*)&tv[rr][cc] = *(const uint4*)(s + r * cols + c);
      }
      __syncthreads();
      for (int e = threadIdx.x; e < 64 * 8; e += 256) {
        const int cc = e / 8, rr = (e % 8) * 8;
        const int64_t r = r0 + rr, c = c0 + cc;
        if (r < rows && c < cols) {
          uint32_t w[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)__builtin_bit_cast(uint16_t, tv[rr + 2 * i][cc]) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, tv[rr + 2 * i + 1][cc]) << 16);
          *(uint4*)(d + c * rows + r) = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
      return;
    }
  }
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int rr = e / 64, cc = e % 64;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (r < rows && c < cols) tile[rr][cc] = s[r * cols + c];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int cc = e / 64, rr = e % 64;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (r < rows && c < cols) d[c * rows + r] = tile[rr][cc];
  }
}

static int blocks_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 8192) b = 8192;
  return (int)(b < 1 ? 1 : b);
}

// Writes [norm, coef] to clip_out. `partials` needs `nparts` floats (nparts <= 8192).
UNOK_EXPORT int unok_grad_clip_coef(int64_t n, const float* g, float* partials, int nparts, float max_norm,
                                    float* clip_out, void* stream) {
  UNOK_REQUIRE(nparts > 0 && nparts <= 8192, UNOK_EINVAL, "grad_clip_coef: nparts=%d outside [1, 8192]", nparts);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(sumsq_kernel, dim3(nparts), dim3(256), 0, st, n, g, partials);
  int rc = unok::check_launch("sumsq");
  if (rc) return rc;
  hipLaunchKernelGGL(clip_coef_kernel, dim3(1), dim3(256), 0, st, nparts, partials, max_norm, clip_out);
  return unok::check_launch("clip_coef");
}

UNOK_EXPORT int unok_adamw_step(int64_t n, float* p, float* g, float* m, float* v, const float* clip, float lr,
                                float beta1, float beta2, float eps, float weight_decay, int step, int copy_dtype,
                                void* copy, int64_t n_unscaled, float copy_scale, void* stream) {
  UNOK_REQUIRE(step >= 1, UNOK_EINVAL, "adamw_step: step must be >= 1 (got %d)", step);
  if (n == 0) return 0;
  AdamArgs a{p, g, m, v, copy, copy_dtype == UNOK_F32, n, n_unscaled, copy_scale, clip, lr, beta1, beta2, eps,
             weight_decay,
             (float)(1.0 - pow((double)beta1, (double)step)), (float)sqrt(1.0 - pow((double)beta2, (double)step))};
  hipLaunchKernelGGL(adamw_kernel, dim3(blocks_for(n)), dim3(256), 0, (hipStream_t)stream, a);
  return unok::check_launch("adamw");
}

UNOK_EXPORT int unok_cast_copy(int copy_dtype, int64_t n, int64_t n_unscaled, float scale, const float* p, void* copy,
                               void* stream) {
  UNOK_REQUIRE(n >= 0 && n_unscaled >= 0, UNOK_EINVAL, "cast_copy: n=%lld n_unscaled=%lld", (long long)n,
               (long long)n_unscaled);
  UNOK_REQUIRE(copy_dtype == UNOK_F32 || copy_dtype == UNOK_BF16, UNOK_EINVAL, "cast_copy: bad dtype %d", copy_dtype);
  if (n == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  if (copy_dtype == UNOK_F32)
    hipLaunchKernelGGL(cast_copy_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, st, n, n_unscaled, scale, p,
                       (float*)copy);
  else
    hipLaunchKernelGGL(cast_copy_kernel<bf16_t>, dim3(blocks_for(n)), dim3(256), 0, st, n, n_unscaled, scale, p,
                       (bf16_t*)copy);
  return unok::check_launch("cast_copy");
}

UNOK_EXPORT int unok_transpose_jobs(int dtype, const int64_t* jobs, int njobs, int64_t total_tiles, const void* src,
                                    void* dst, void* stream) {
  UNOK_REQUIRE(njobs >= 0 && total_tiles >= 0 && total_tiles <= 0xFFFFFFFFll, UNOK_EINVAL,
               "transpose_jobs: njobs=%d total_tiles=%lld", njobs, (long long)total_tiles);
  UNOK_REQUIRE(dtype == UNOK_F32 || dtype == UNOK_BF16, UNOK_EINVAL, "transpose_jobs: bad dtype %d", dtype);
  if (njobs == 0 || total_tiles == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == UNOK_F32)
    hipLaunchKernelGGL(transpose_jobs_kernel<float>, dim3((unsigned)total_tiles), dim3(256), 0, st, jobs, njobs,
                       (const float*)src, (float*)dst);
  else
    hipLaunchKernelGGL(transpose_jobs_kernel<bf16_t>, dim3((unsigned)total_tiles), dim3(256), 0, st, jobs, njobs,
                       (const bf16_t*)src, (bf16_t*)dst);
  return unok::check_launch("transpose_jobs");
}
