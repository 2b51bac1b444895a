// Weight formats as seen by the wave64 matrix-vector kernels.
//
// A row is cut into "units" of consecutive weights; a lane owns whole units.
// Each format provides
//   kUnit          weights per unit
//   Frag           the lane's inputs for one unit, in registers
//   load(x, nw, u) the inputs of unit u, times the norm weights when given
//   dot(row, u, f) the unit's part of the row's dot product
// The Q4_K unit is one pair of 32-element blocks of a 144-byte super-block:
// 32 bytes of quants (low nibbles = block 2p, high nibbles = block 2p+1)
// plus the 16-byte header (fp16 d, fp16 dmin, 12 scale bytes).  A lane
// therefore issues three 16-byte loads per 64 weights and keeps its 64
// inputs in VGPRs while it walks rows.
#pragma once
#include "device.h"

namespace bch {

// Element `col` of a row of `format` at `row`, dequantised exactly as
// scalar::dequantize (crates/bobcat/src/scalar.rs:59-202): every product
// rounds on its own (no contraction).
__device__ __forceinline__ float dequant_elem(uint32_t format, const uint8_t *row, uint32_t col) {
  switch (format) {
    case 0: return reinterpret_cast<const float *>(row)[col];
    case 1: return half_bits_to_float(reinterpret_cast<const uint16_t *>(row)[col]);
    case 30: return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(row)[col] << 16);
    case 2: {  // Q4_0 (scalar.rs:95-104)
      const uint8_t *b = row + (col / 32) * 18;
      const uint32_t i = col % 32;
      const float d = half_bits_to_float(b[0] | (b[1] << 8));
      const uint8_t q = b[2 + (i % 16)];
      const int v = (i < 16 ? (q & 0xf) : (q >> 4)) - 8;
      return __fmul_rn((float)v, d);
    }
    case 8: {  // Q8_0 (scalar.rs:107-112)
      const uint8_t *b = row + (col / 32) * 34;
      const float d = half_bits_to_float(b[0] | (b[1] << 8));
      return __fmul_rn((float)(int8_t)b[2 + col % 32], d);
    }
    case 12: {  // Q4_K (scalar.rs:127-152)
      const uint8_t *b = row + (col / 256) * 144;
      const uint32_t i = col % 256, j = i / 32, l = i % 32;
      const float d = half_bits_to_float(b[0] | (b[1] << 8));
      const float dmin = half_bits_to_float(b[2] | (b[3] << 8));
      const uint8_t *s = b + 4;
      uint32_t sc, mn;
      if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
      } else {
        sc = (s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
      }
      const uint8_t q = b[16 + 32 * (j / 2) + l];
      const uint32_t nib = (j & 1) ? (q >> 4) : (q & 0xf);
      return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)nib), __fmul_rn(dmin, (float)mn));
    }
    case 13: {  // Q5_K (scalar.rs:157-176)
      const uint8_t *b = row + (col / 256) * 176;
      const uint32_t i = col % 256, j = i / 32, l = i % 32;
      const float d = half_bits_to_float(b[0] | (b[1] << 8));
      const float dmin = half_bits_to_float(b[2] | (b[3] << 8));
      const uint8_t *s = b + 4;
      uint32_t sc, mn;
      if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
      } else {
        sc = (s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
      }
      const uint8_t q = b[48 + 32 * (j / 2) + l];
      const uint32_t v = ((q >> (4 * (j % 2))) & 0xf) | (((b[16 + l] >> j) & 1) << 4);
      return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)v), __fmul_rn(dmin, (float)mn));
    }
    case 14: {  // Q6_K (scalar.rs:181-202)
      const uint8_t *b = row + (col / 256) * 210;
      const uint32_t i = col % 256, half = i / 128, r = i % 128, quarter = r / 32, l = r % 32;
      const float d = half_bits_to_float(b[208] | (b[209] << 8));
      const uint8_t *low = b + half * 64, *high = b + 128 + half * 32;
      const int8_t *sc = reinterpret_cast<const int8_t *>(b + 192 + half * 8);
      const uint32_t lb = (quarter & 1) ? low[l + 32] : low[l];
      const uint32_t lo = (quarter < 2) ? (lb & 0xf) : (lb >> 4);
      const uint32_t hi = (high[l] >> (2 * quarter)) & 3;
      const int q = (int)(lo | (hi << 4)) - 32;
      const float scale = __fmul_rn(d, (float)sc[l / 16 + 2 * quarter]);
      return __fmul_rn(scale, (float)q);
    }
  }
  return 0.f;
}

template <bool NORM>
__device__ __forceinline__ void load_inputs(const float *__restrict__ x, const float *__restrict__ nw,
                                            uint32_t first, float *out, int n4) {
  const float4 *xp = reinterpret_cast<const float4 *>(x + first);
#pragma unroll
  for (int i = 0; i < n4; i++) {
    float4 v = xp[i];
    if (NORM) {
      const float4 w = reinterpret_cast<const float4 *>(nw + first)[i];
      v.x *= w.x;
      v.y *= w.y;
      v.z *= w.z;
      v.w *= w.w;
    }
    out[4 * i + 0] = v.x;
    out[4 * i + 1] = v.y;
    out[4 * i + 2] = v.z;
    out[4 * i + 3] = v.w;
  }
}

struct Q4K {
  static constexpr uint32_t kFormat = 12;
  static constexpr uint32_t kUnit = 64;
  struct Frag {
    float lo[32];  // inputs of block 2p
    float hi[32];  // inputs of block 2p+1
    float sum_lo, sum_hi;
  };
  template <bool NORM>
  __device__ __forceinline__ static void load(const float *x, const float *nw, uint32_t u, Frag &f) {
    const uint32_t first = (u >> 2) * 256 + (u & 3) * 64;
    load_inputs<NORM>(x, nw, first, f.lo, 8);
    load_inputs<NORM>(x, nw, first + 32, f.hi, 8);
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      a += f.lo[i];
      b += f.hi[i];
    }
    f.sum_lo = a;
    f.sum_hi = b;
  }
  // The unit's inputs from 64 consecutive floats (16-byte aligned, in LDS).
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) {
    const float4 *p4 = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 a = p4[i], b = p4[8 + i];
      f.lo[4 * i] = a.x, f.lo[4 * i + 1] = a.y, f.lo[4 * i + 2] = a.z, f.lo[4 * i + 3] = a.w;
      f.hi[4 * i] = b.x, f.hi[4 * i + 1] = b.y, f.hi[4 * i + 2] = b.z, f.hi[4 * i + 3] = b.w;
    }
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      sa += f.lo[i];
      sb += f.hi[i];
    }
    f.sum_lo = sa;
    f.sum_hi = sb;
  }
  // d·(sc_lo·Σq·x + sc_hi·Σq'·x') − dmin·(m_lo·Σx + m_hi·Σx'), which is
  // Σ_l ((d·sc)·q_l − dmin·m)·x_l regrouped.
  // The unit's 48 bytes: the super-block header and the pair's 32 quant bytes.
  struct Raw {
    uint4 h, q0, q1;
  };
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) {
    const uint8_t *blk = row + (u >> 2) * 144;
    const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 16 + 32 * (u & 3));
    return Raw{*reinterpret_cast<const uint4 *>(blk), qp[0], qp[1]};
  }
  __device__ __forceinline__ static float dot(const uint8_t *__restrict__ row, uint32_t u, const Frag &f) {
    return compute(fetch(row, u), u, f);
  }
  __device__ __forceinline__ static float compute(const Raw &raw, uint32_t u, const Frag &f) {
    const int p = u & 3;
    const uint4 h = raw.h, q0 = raw.q0, q1 = raw.q1;
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    float s_lo0 = 0.f, s_lo1 = 0.f, s_hi0 = 0.f, s_hi1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t lo = qw[k] & 0x0f0f0f0fu;
      const uint32_t hi = (qw[k] >> 4) & 0x0f0f0f0fu;
      s_lo0 = fmaf(ubyte0(lo), f.lo[4 * k + 0], s_lo0);
      s_lo1 = fmaf(ubyte1(lo), f.lo[4 * k + 1], s_lo1);
      s_lo0 = fmaf(ubyte2(lo), f.lo[4 * k + 2], s_lo0);
      s_lo1 = fmaf(ubyte3(lo), f.lo[4 * k + 3], s_lo1);
      s_hi0 = fmaf(ubyte0(hi), f.hi[4 * k + 0], s_hi0);
      s_hi1 = fmaf(ubyte1(hi), f.hi[4 * k + 1], s_hi1);
      s_hi0 = fmaf(ubyte2(hi), f.hi[4 * k + 2], s_hi0);
      s_hi1 = fmaf(ubyte3(hi), f.hi[4 * k + 3], s_hi1);
    }
    const uint32_t sc = q4k_pair_scales(h.y, h.z, h.w, p);
    const float d = half_bits_to_float(h.x & 0xffffu);
    const float dmin = half_bits_to_float(h.x >> 16);
    const float qs = ubyte0(sc) * (s_lo0 + s_lo1) + ubyte1(sc) * (s_hi0 + s_hi1);
    const float ms = ubyte2(sc) * f.sum_lo + ubyte3(sc) * f.sum_hi;
    return d * qs - dmin * ms;
  }
};

struct F16 {
  static constexpr uint32_t kFormat = 1;
  static constexpr uint32_t kUnit = 8;
  struct Frag {
    float x[8];
  };
  template <bool NORM>
  __device__ __forceinline__ static void load(const float *x, const float *nw, uint32_t u, Frag &f) {
    load_inputs<NORM>(x, nw, u * 8, f.x, 2);
  }
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    f.x[0] = a.x, f.x[1] = a.y, f.x[2] = a.z, f.x[3] = a.w, f.x[4] = b.x, f.x[5] = b.y, f.x[6] = b.z, f.x[7] = b.w;
  }
  using Raw = uint4;
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) {
    return reinterpret_cast<const uint4 *>(row)[u];
  }
  __device__ __forceinline__ static float dot(const uint8_t *__restrict__ row, uint32_t u, const Frag &f) {
    return compute(fetch(row, u), u, f);
  }
  __device__ __forceinline__ static float compute(const Raw &w, uint32_t, const Frag &f) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      s0 = fmaf(half_bits_to_float(ws[k] & 0xffffu), f.x[2 * k], s0);
      s1 = fmaf(half_bits_to_float(ws[k] >> 16), f.x[2 * k + 1], s1);
    }
    return s0 + s1;
  }
};

struct F32 {
  static constexpr uint32_t kFormat = 0;
  static constexpr uint32_t kUnit = 4;
  struct Frag {
    float x[4];
  };
  template <bool NORM>
  __device__ __forceinline__ static void load(const float *x, const float *nw, uint32_t u, Frag &f) {
    load_inputs<NORM>(x, nw, u * 4, f.x, 1);
  }
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    f.x[0] = a.x, f.x[1] = a.y, f.x[2] = a.z, f.x[3] = a.w;
  }
  using Raw = float4;
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) {
    return reinterpret_cast<const float4 *>(row)[u];
  }
  __device__ __forceinline__ static float dot(const uint8_t *__restrict__ row, uint32_t u, const Frag &f) {
    return compute(fetch(row, u), u, f);
  }
  __device__ __forceinline__ static float compute(const Raw &w, uint32_t, const Frag &f) {
    return fmaf(w.x, f.x[0], w.y * f.x[1]) + fmaf(w.z, f.x[2], w.w * f.x[3]);
  }
};

}  // namespace bch
