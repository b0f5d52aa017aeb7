// Block-diffusion batch preparation on the device: per-token noising with counter-based
// splitmix64 draws, the [noisy | clean] per-segment concatenation, the stream maps between the
// concatenated layout and the two stream layouts, and the attention interval tables.
//
// Contract (shared bit-for-bit with the CPU oracle):
//   segments start at t = 0 and wherever pos[t-1] >= pos[t];
//   block(j) = j / block_size for in-segment index j;
//   key = mix64(seed + GOLDEN*(step+1));
//   draw(stream, row, idx) = mix64(mix64(mix64(key ^ stream) + row*GOLDEN) + idx*GOLDEN);
//   t(block) = fl32(fl32(u * 0.95f) + 0.05f), u = (draw(1, b, s + block*bs) >> 40) * 2^-24;
//   noised iff !prompt && (draw(2, b, t) >> 40) * 2^-24 < t(block);
//   uniform noise id = 1 + draw(3, b, t) mod (mask_id - 1); mask noise id = mask_id.
// mix64 is the splitmix64 finaliser (nano_vllm_uno/engine/noise.py:43-50).
#include "common.h"

// Floating-point contraction is off in this file: the noise level is specified as two
// separately rounded fp32 operations, which a fused multiply-add would merge into one.
#pragma clang fp contract(off)

#define GOLDEN 0x9E3779B97F4A7C15ull

__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ uint64_t draw(uint64_t key, uint64_t stream, uint64_t row, uint64_t idx) {
  return mix64(mix64(mix64(key ^ stream) + row * GOLDEN) + idx * GOLDEN);
}

__device__ __forceinline__ float unit24(uint64_t h) { return (float)(uint32_t)(h >> 40) * 5.9604644775390625e-8f; }

// t = fl32(fl32(u * 0.95f) + 0.05f). Plain operators on purpose: this file is compiled with
// contraction off, whereas HIP's __fmul_rn/__fadd_rn are header inlines that still fuse.
__device__ __forceinline__ float noise_level(float u) {
  const float scaled = u * 0.95f;
  return scaled + 0.05f;
}

struct BdArgs {
  const int64_t* ids; const int64_t* pos; const uint8_t* prompt;
  int B, L, bs, mask_id, noise_mask_mode, intra_causal;
  uint64_t key;
  // outputs
  int64_t* concat_ids; int64_t* concat_pos; uint8_t* region;  // [B, 2L]
  uint8_t* noised; float* tfull;                               // [B, L]
  int32_t* noisy_src; int32_t* clean_src;                      // [B*L] concat flat indices
  int32_t* noisy_iv; int32_t* clean_iv;                        // [B*L, 8]
  int64_t* noisy_ids; int64_t* clean_ids;                      // [B*L] token ids per stream row
};

// One workgroup per batch row. Segment starts/ends come from a chunked scan. REGION_ONLY writes
// just the [noisy | clean] region mask (the layout step that precedes noising).
template <bool REGION_ONLY>
__global__ __launch_bounds__(1024) void bd_prepare_kernel(const BdArgs a) {
  __shared__ int carry_start[1024];
  __shared__ int carry_end[1024];
  const int b = blockIdx.x, L = a.L, tid = threadIdx.x;
  const int chunk = (L + 1023) / 1024;
  const int c0 = min(L, tid * chunk), c1 = min(L, c0 + chunk);
  const int64_t* pos = a.pos + (int64_t)b * L;
  int last_start = -1, first_start = INT_MAX;
  for (int t = c0; t < c1; ++t) {
    const bool st = (t == 0) || (pos[t - 1] >= pos[t]);
    if (st) { last_start = t; if (first_start == INT_MAX) first_start = t; }
  }
  carry_start[tid] = last_start;
  carry_end[tid] = first_start;
  __syncthreads();
  if (tid == 0) {
    int run = -1;
    for (int i = 0; i < 1024; ++i) { const int v = carry_start[i]; carry_start[i] = run; if (v > run) run = v; }
    int runm = L;
    for (int i = 1023; i >= 0; --i) { const int v = carry_end[i]; carry_end[i] = runm; if (v < runm) runm = v; }
  }
  __syncthreads();
  // carry_start[i]: last segment start before chunk i; carry_end[i]: first start after chunk i.
  // Within a chunk (L/1024 tokens) the next start is found by a short forward walk.
  int seg_s = carry_start[tid];
  const int next_start = carry_end[tid];
  for (int t = c0; t < c1; ++t) {
    const bool st = (t == 0) || (pos[t - 1] >= pos[t]);
    if (st) seg_s = t;
    // segment end: first start > t
    int e = next_start;
    for (int u = t + 1; u < c1; ++u)
      if (pos[u - 1] >= pos[u]) { e = u; break; }
    const int64_t base2 = (int64_t)b * 2 * L;
    if (REGION_ONLY) {
      a.region[base2 + seg_s + t] = 1;
      a.region[base2 + e + t] = 0;
      continue;
    }
    const int s = seg_s, len = e - s, j = t - s, blk = j / a.bs;
    const int bstart = s + blk * a.bs;
    const int bend = min(bstart + a.bs, e);
    const int64_t gi = (int64_t)b * L + t;
    const float u_blk = unit24(draw(a.key, 1, (uint64_t)b, (uint64_t)bstart));
    const float tb = noise_level(u_blk);
    const float u_tok = unit24(draw(a.key, 2, (uint64_t)b, (uint64_t)t));
    const bool noised = !a.prompt[gi] && (u_tok < tb);
    const int64_t id = a.ids[gi];
    int64_t nid = id;
    if (noised) {
      if (a.noise_mask_mode) nid = a.mask_id;
      else nid = 1 + (int64_t)(draw(a.key, 3, (uint64_t)b, (uint64_t)t) % (uint64_t)(a.mask_id - 1));
    }
    a.noised[gi] = noised ? 1 : 0;
    a.tfull[gi] = tb;
    const int64_t nidx = base2 + s + t, cidx = base2 + e + t;
    a.concat_ids[nidx] = nid;
    a.concat_ids[cidx] = id;
    a.concat_pos[nidx] = pos[t];
    a.concat_pos[cidx] = pos[t];
    a.region[nidx] = 1;
    a.region[cidx] = 0;
    a.noisy_src[gi] = (int32_t)nidx;
    a.clean_src[gi] = (int32_t)cidx;
    a.noisy_ids[gi] = nid;
    a.clean_ids[gi] = id;
    const int base = b * L;
    int32_t* nv = a.noisy_iv + gi * 8;
    int32_t* cv = a.clean_iv + gi * 8;
    nv[0] = base + s;
    nv[1] = base + bstart;
    nv[2] = base + bstart;
    nv[3] = a.intra_causal ? base + t + 1 : base + bend;
    nv[4] = a.intra_causal ? base + t : base + bstart;
    nv[5] = base + bend;
    nv[6] = 0;
    nv[7] = len;
    cv[0] = base + s;
    cv[1] = base + t + 1;
    cv[2] = 0; cv[3] = 0; cv[4] = 0; cv[5] = 0; cv[6] = 0;
    cv[7] = len;
  }
}

// p_mask compaction over the row-major [B*L] noised flags (single workgroup, chunked scan); with
// positions, also their maximum (clamped to [0, 2^31 - 1]) into count[1], read back with the count.
__global__ __launch_bounds__(1024) void bd_compact_kernel(const uint8_t* __restrict__ noised,
                                                          const float* __restrict__ tfull,
                                                          const int64_t* __restrict__ pos, int64_t n,
                                                          float* __restrict__ p_mask, int32_t* __restrict__ count) {
  __shared__ int32_t part[1024];
  __shared__ int64_t pmax[1024];
  const int tid = threadIdx.x;
  const int64_t chunk = (n + 1023) / 1024;
  const int64_t c0 = min(n, tid * chunk), c1 = min(n, c0 + chunk);
  int32_t cnt = 0;
  int64_t mx = 0;
  for (int64_t i = c0; i < c1; ++i) cnt += noised[i] ? 1 : 0;
  if (pos)
    for (int64_t i = c0; i < c1; ++i) mx = max(mx, pos[i]);
  part[tid] = cnt;
  pmax[tid] = mx;
  __syncthreads();
  if (tid == 0) {
    int32_t run = 0;
    int64_t m = 0;
    for (int i = 0; i < 1024; ++i) { const int32_t v = part[i]; part[i] = run; run += v; m = max(m, pmax[i]); }
    count[0] = run;
    if (pos) count[1] = (int32_t)min(m, (int64_t)0x7fffffff);
  }
  __syncthreads();
  int32_t o = part[tid];
  for (int64_t i = c0; i < c1; ++i)
    if (noised[i]) p_mask[o++] = tfull[i];
}

UNOK_EXPORT int unok_bd_prepare(int B, int L, const int64_t* ids, const int64_t* pos, const uint8_t* prompt,
                                int block_size, int mask_id, int noise_mask_mode, int intra_causal, uint64_t key,
                                int64_t* concat_ids, int64_t* concat_pos, uint8_t* region, uint8_t* noised,
                                float* tfull, int32_t* noisy_src, int32_t* clean_src, int32_t* noisy_iv,
                                int32_t* clean_iv, int64_t* noisy_ids, int64_t* clean_ids, void* stream) {
  UNOK_REQUIRE(B >= 0 && L >= 0, UNOK_EINVAL, "bd_prepare: negative shape");
  if (B == 0 || L == 0) return 0;
  UNOK_REQUIRE(block_size > 0, UNOK_EINVAL, "bd_prepare: block_size must be positive (got %d)", block_size);
  UNOK_REQUIRE(mask_id > 1, UNOK_EINVAL, "bd_prepare: mask_token_id must be > 1 (got %d)", mask_id);
  UNOK_REQUIRE((int64_t)B * 2 * L < INT32_MAX, UNOK_EINVAL, "bd_prepare: batch too large for int32 maps");
  BdArgs a{ids, pos, prompt, B, L, block_size, mask_id, noise_mask_mode, intra_causal, key,
           concat_ids, concat_pos, region, noised, tfull, noisy_src, clean_src, noisy_iv, clean_iv, noisy_ids,
           clean_ids};
  hipLaunchKernelGGL(bd_prepare_kernel<false>, dim3(B), dim3(1024), 0, (hipStream_t)stream, a);
  return unok::check_launch("bd_prepare");
}

UNOK_EXPORT int unok_bd_region(int B, int L, const int64_t* pos, uint8_t* region, void* stream) {
  UNOK_REQUIRE(B >= 0 && L >= 0, UNOK_EINVAL, "bd_region: negative shape");
  if (B == 0 || L == 0) return 0;
  UNOK_REQUIRE((int64_t)B * 2 * L < INT32_MAX, UNOK_EINVAL, "bd_region: batch too large");
  BdArgs a{};
  a.pos = pos; a.B = B; a.L = L; a.bs = 1; a.region = region;
  hipLaunchKernelGGL(bd_prepare_kernel<true>, dim3(B), dim3(1024), 0, (hipStream_t)stream, a);
  return unok::check_launch("bd_region");
}

UNOK_EXPORT int unok_bd_compact(int64_t n, const uint8_t* noised, const float* tfull, const int64_t* pos,
                                float* p_mask, int32_t* count, void* stream) {
  UNOK_REQUIRE(n >= 0, UNOK_EINVAL, "bd_compact: negative size");
  hipLaunchKernelGGL(bd_compact_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, noised, tfull, pos, n, p_mask,
                     count);
  return unok::check_launch("bd_compact");
}
