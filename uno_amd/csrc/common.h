// Shared device helpers and C-ABI error plumbing for the uno_amd kernel library.
//
// Conventions used by every entry point in this library:
//   * every exported function is `extern "C" int unok_*(...)`, returns 0 on success,
//     a positive hipError_t on a launch failure, or a negative code for argument errors;
//   * the message for the last failure on the calling thread is kept in a thread-local
//     buffer and returned by unok_last_error();
//   * tensors are raw device pointers with explicit element strides; the caller (PyTorch)
//     owns every allocation, and all work is enqueued on the hipStream_t it passes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#define UNOK_EXPORT extern "C" __attribute__((visibility("default")))

// dtype codes shared with the Python side.
enum UnokDtype : int { UNOK_F32 = 0, UNOK_BF16 = 1 };

// Negative return codes for argument errors.
enum UnokArgError : int {
  UNOK_EINVAL = -1,     // bad size / stride / dtype combination
  UNOK_EALIGN = -2,     // pointer or stride alignment requirement violated
  UNOK_EUNSUPPORTED = -3,
};

namespace unok {

int set_error(int code, const char* fmt, ...);
const char* last_error();

// Converts a hipError_t from a launch into the return convention above.
int check_launch(const char* what);

}  // namespace unok

#define UNOK_REQUIRE(cond, code, ...)                 \
  do {                                                \
    if (!(cond)) return unok::set_error((code), __VA_ARGS__); \
  } while (0)

// Raises a kernel's dynamic-LDS limit once per process. The function-local static is initialised
// under the C++ runtime's guard, so concurrent first launches from the autograd worker thread and
// the main thread are safe.
#define UNOK_SET_LDS_ONCE(kernel, bytes)                                                                \
  do {                                                                                                  \
    static const bool lds_set_ = [] {                                                                   \
      (void)hipFuncSetAttribute((const void*)(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, (int)(bytes)); \
      return true;                                                                                      \
    }();                                                                                                \
    (void)lds_set_;                                                                                     \
  } while (0)

// ---------------------------------------------------------------------------------------
// bf16 helpers. bf16 values travel as uint16_t bit patterns; conversions use
// round-to-nearest-even, the rounding torch uses for float -> bfloat16.
// ---------------------------------------------------------------------------------------
typedef uint16_t bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even conversion in hardware (v_cvt_pk_bf16_f32 on gfx950); NaN stays NaN.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return (bf16_t)(pack2_bf16(f, 0.f) & 0xffffu); }

// Generic element load/store used by kernels templated on the storage type.
template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
  // Value after a round trip through the storage type.
  __device__ __forceinline__ static float round(float v) { return v; }
};
template <> struct Elem<bf16_t> {
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
  __device__ __forceinline__ static float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};

// 64-lane wavefront reductions (CDNA wavefronts are 64 wide).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Block-wide sum for blocks of up to 1024 threads; `red` needs 32 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = (threadIdx.x < (unsigned)nw) ? red[threadIdx.x] : 0.f;
  if (wid == 0) t = wave_sum(t);
  if (threadIdx.x == 0) red[0] = t;
  __syncthreads();
  float r = red[0];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = (threadIdx.x < (unsigned)nw) ? red[threadIdx.x] : -INFINITY;
  if (wid == 0) t = wave_max(t);
  if (threadIdx.x == 0) red[0] = t;
  __syncthreads();
  float r = red[0];
  __syncthreads();
  return r;
}

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32, within 1 ulp; results below the normal
// range flush to zero). Used where x <= 0 or the result only enters a sum or a ratio: softmax
// weights of the loss kernels and the logistic function below.
__device__ __forceinline__ float fast_expf(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// Logistic function of the SwiGLU gate, 1 / (1 + e^-g) with the hardware reciprocal (within
// 1 ulp); +-inf give 0 and 1. One definition, so the fused GEMM epilogues and the stand-alone
// SwiGLU kernels round identically.
__device__ __forceinline__ float sigmoidf_(float g) { return __builtin_amdgcn_rcpf(1.f + fast_expf(-g)); }

// Gradients of out = silu(g) * u for upstream d: the same expression in the SwiGLU backward kernel
// and the fused GEMM epilogue, so both round identically.
__device__ __forceinline__ void swiglu_grad(float d, float g, float u, float& dg, float& du) {
  const float sg = sigmoidf_(g);
  du = d * (g * sg);
  dg = d * u * sg * (1.f + g * (1.f - sg));
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int SG_VALU = 0x002, SG_MFMA = 0x008, SG_VMEM = 0x010, SG_DS_READ = 0x100;

// Maps a linear workgroup id so that consecutive logical tiles land on the same XCD.
// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X; grouping logical
// neighbours on one XCD lets them share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int NXCD = 8;
  const int full = nblocks - nblocks % NXCD;
  if (bid >= full) return bid;
  const int per = full / NXCD;
  return (bid % NXCD) * per + bid / NXCD;
}
