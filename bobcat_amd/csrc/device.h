// Device helpers shared by the gfx950 kernels: wave64 reductions, half
// conversion, and the Q4_K super-block decoder.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace bch {

constexpr int kWave = 64;

// DPP lane moves within rows of 16 lanes: the source lane of each lane.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141; // 7 - lane within each 8 lanes
constexpr int kDppMirror = 0x140;     // 15 - lane within each 16 lanes
constexpr int kDppRor4 = 0x124;       // (lane + 4) % 16 within the row
constexpr int kDppRor8 = 0x128;       // (lane + 8) % 16 within the row

// `v` of the lane that DPP control CTRL names.  All lanes of the row must
// be active (callers use these in code that whole rows execute together).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum of `v` over groups of `width` consecutive lanes (width a power of two
// up to 64); every lane of a group receives the group's sum.  The tree
// pairs neighbouring lanes first: quads by DPP quad permutes, eights and
// sixteens by the DPP mirrors (lane i and its mirror lie in the two halves),
// and across rows by a lane shuffle.  Each step adds two group sums, so all
// lanes of a group hold the same value.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (width >= 2) v += dpp<kDppXor1>(v);
  if constexpr (width >= 4) v += dpp<kDppXor2>(v);
  if constexpr (width >= 8) v += dpp<kDppHalfMirror>(v);
  if constexpr (width >= 16) v += dpp<kDppMirror>(v);
  if constexpr (width >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (width >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}

// Sum over a workgroup of `threads` threads; `scratch` holds threads/64
// floats.  Every thread receives the total.
template <int threads>
__device__ __forceinline__ float block_sum(float v, float *scratch) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (threads > kWave) {
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < threads / kWave; w++) t += scratch[w];
    __syncthreads();
    return t;
  }
  return v;
}

// Maximum over a workgroup of `threads` threads (scratch as block_sum).
template <int threads>
__device__ __forceinline__ float block_max(float v, float *scratch) {
  v = wave_max(v);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (threads > kWave) {
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = -INFINITY;
#pragma unroll
    for (int w = 0; w < threads / kWave; w++) t = fmaxf(t, scratch[w]);
    __syncthreads();
    return t;
  }
  return v;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)bits16));
}

// Byte k of a dword as a float (v_cvt_f32_ubyte{k}).  Written as inline
// asm so that a masked dword feeds all four conversions directly; plain C
// makes the compiler insert a v_bfe_u32 before each conversion.
__device__ __forceinline__ float ubyte0(uint32_t w) {
  float r;
  asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
  return r;
}
__device__ __forceinline__ float ubyte1(uint32_t w) {
  float r;
  asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
  return r;
}
__device__ __forceinline__ float ubyte2(uint32_t w) {
  float r;
  asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
  return r;
}
__device__ __forceinline__ float ubyte3(uint32_t w) {
  float r;
  asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
  return r;
}

// The 6-bit scales and minimums of 32-element blocks 2p and 2p+1 of a Q4_K
// super-block, packed as bytes (scale_2p, scale_2p+1, min_2p, min_2p+1).
// h1, h2, h3 are header dwords 1..3 (the 12 scale bytes s[0..11]).  The
// unpacking is q4k_scale_min (crates/bobcat/src/scalar.rs:116-125) for
// two blocks at once.
__device__ __forceinline__ uint32_t q4k_pair_scales(uint32_t h1, uint32_t h2, uint32_t h3, int p) {
  const int sh = 16 * (p & 1);
  const uint32_t a = (h1 >> sh) & 0xffffu;  // s[2p'], s[2p'+1] with p' = p & 1
  const uint32_t b = (h2 >> sh) & 0xffffu;  // s[2p'+4], s[2p'+5]
  const uint32_t c = (h3 >> sh) & 0xffffu;  // s[2p+4], s[2p+5] for p >= 2
  // Both cases are computed and selected without a branch: a lane-dependent
  // branch here would make the last header dword a divergent load.
  const uint32_t low = (a & 0x3f3fu) | ((b & 0x3f3fu) << 16);
  const uint32_t sc = (c & 0x0f0fu) | ((a >> 2) & 0x3030u);
  const uint32_t mn = ((c >> 4) & 0x0f0fu) | ((b >> 2) & 0x3030u);
  const uint32_t high = sc | (mn << 16);
  return p < 2 ? low : high;
}

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load of the wave (s_waitcnt vmcnt(0)), which
// would hold a kernel that has its weight loads in flight until all of them
// have arrived; this barrier lets those loads keep streaming.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Device-scope relaxed accesses for data one workgroup hands to another on
// any XCD (they go past the non-coherent L2 of the writer's XCD).
template <class T>
__device__ __forceinline__ void coherent_store(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T coherent_load(const T *p) {
  return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace bch
