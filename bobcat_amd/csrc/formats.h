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

// --- the other GGUF formats of real Q4_K_M / Q4_0 / Q8_0 files ------------
//
// A 64-weight unit of these formats is not 16-byte aligned (Q8_0 blocks are
// 34 bytes, Q4_0 18, Q6_K super-blocks 210), so a unit is read as dwords
// from the dword at or below its first byte and realigned with alignbyte.

// n dwords starting at byte address p (2-byte aligned), via aligned loads;
// the dword past the last one is read only when p is not dword aligned (its
// first two bytes are then still the caller's), so nothing past p + 4n + 1
// is touched.
template <int N>
__device__ __forceinline__ void load_dwords(const uint8_t *p, uint32_t *out) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t *w = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
  const uint32_t sh = (uint32_t)(a & 3);
  uint32_t raw[N + 1];
#pragma unroll
  for (int i = 0; i < N; i++) raw[i] = w[i];
  raw[N] = sh ? w[N] : 0u;
#pragma unroll
  for (int i = 0; i < N; i++) out[i] = sh ? __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh) : raw[i];
}

// The inputs of a 64-weight unit: the values and the sums of its four
// 16-element groups.
struct Frag64 {
  float x[64];
  float gs[4];
};

__device__ __forceinline__ void frag64_from_lds(const float *p, Frag64 &f) {
  const float4 *p4 = reinterpret_cast<const float4 *>(p);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const float4 a = p4[i];
    f.x[4 * i] = a.x, f.x[4 * i + 1] = a.y, f.x[4 * i + 2] = a.z, f.x[4 * i + 3] = a.w;
  }
#pragma unroll
  for (int g = 0; g < 4; g++) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) t += f.x[16 * g + i];
    f.gs[g] = t;
  }
}

template <bool NORM>
__device__ __forceinline__ void frag64_load(const float *x, const float *nw, uint32_t u, Frag64 &f) {
  load_inputs<NORM>(x, nw, u * 64, f.x, 16);
#pragma unroll
  for (int g = 0; g < 4; g++) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) t += f.x[16 * g + i];
    f.gs[g] = t;
  }
}

// Σ over 4 bytes of dword w (unsigned) times x[0..3].
__device__ __forceinline__ float dot4u(uint32_t w, const float *x, float acc) {
  acc = fmaf(ubyte0(w), x[0], acc);
  acc = fmaf(ubyte1(w), x[1], acc);
  acc = fmaf(ubyte2(w), x[2], acc);
  return fmaf(ubyte3(w), x[3], acc);
}

// Q8_0 (scalar.rs:106-113): 32-weight blocks of fp16 d and 32 int8; a unit
// is two blocks (68 bytes).  Σ d·q·x = d·(Σ (q+128)·x − 128·Σx): the bytes
// flipped to unsigned feed v_cvt_f32_ubyte directly.
struct Q8_0 {
  static constexpr uint32_t kFormat = 8;
  static constexpr uint32_t kUnit = 64;
  using Frag = Frag64;
  template <bool NORM>
  __device__ __forceinline__ static void load(const float *x, const float *nw, uint32_t u, Frag &f) {
    frag64_load<NORM>(x, nw, u, f);
  }
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) { frag64_from_lds(p, f); }
  struct Raw {
    uint32_t w[17];
  };
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) {
    Raw r;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row + 68 * u);
#pragma unroll
    for (int i = 0; i < 17; i++) r.w[i] = p[i];
    return r;
  }
  __device__ __forceinline__ static float compute(const Raw &r, uint32_t, const Frag &f) {
    float tot = 0.f;
#pragma unroll
    for (int b = 0; b < 2; b++) {
      // Block b: d at byte 34b, quants at bytes 34b+2 .. 34b+33.
      const float d = half_bits_to_float(b == 0 ? (r.w[0] & 0xffffu) : (r.w[8] >> 16));
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t q = b == 0 ? __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2) : r.w[9 + i];
        const float *x = f.x + 32 * b + 4 * i;
        if (i & 1)
          s1 = dot4u(q ^ 0x80808080u, x, s1);
        else
          s0 = dot4u(q ^ 0x80808080u, x, s0);
      }
      tot = fmaf(d, (s0 + s1) - 128.f * (f.gs[2 * b] + f.gs[2 * b + 1]), tot);
    }
    return tot;
  }
  __device__ __forceinline__ static float dot(const uint8_t *__restrict__ row, uint32_t u, const Frag &f) {
    return compute(fetch(row, u), u, f);
  }
};

// Q4_0 (scalar.rs:95-104): 32-weight blocks of fp16 d and 16 bytes, low
// nibbles elements 0..15 and high nibbles 16..31, value (q − 8)·d; a unit is
// two blocks (36 bytes).
struct Q4_0 {
  static constexpr uint32_t kFormat = 2;
  static constexpr uint32_t kUnit = 64;
  using Frag = Frag64;
  template <bool NORM>
  __device__ __forceinline__ static void load(const float *x, const float *nw, uint32_t u, Frag &f) {
    frag64_load<NORM>(x, nw, u, f);
  }
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) { frag64_from_lds(p, f); }
  struct Raw {
    uint32_t w[9];
  };
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) {
    Raw r;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row + 36 * u);
#pragma unroll
    for (int i = 0; i < 9; i++) r.w[i] = p[i];
    return r;
  }
  __device__ __forceinline__ static float compute(const Raw &r, uint32_t, const Frag &f) {
    float tot = 0.f;
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const float d = half_bits_to_float(b == 0 ? (r.w[0] & 0xffffu) : (r.w[4] >> 16));
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t q = b == 0 ? __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2) : r.w[5 + i];
        s0 = dot4u(q & 0x0f0f0f0fu, f.x + 32 * b + 4 * i, s0);
        s1 = dot4u((q >> 4) & 0x0f0f0f0fu, f.x + 32 * b + 16 + 4 * i, s1);
      }
      tot = fmaf(d, (s0 + s1) - 8.f * (f.gs[2 * b] + f.gs[2 * b + 1]), tot);
    }
    return tot;
  }
  __device__ __forceinline__ static float dot(const uint8_t *__restrict__ row, uint32_t u, const Frag &f) {
    return compute(fetch(row, u), u, f);
  }
};

// Q6_K (scalar.rs:181-202): 256-weight super-blocks of 210 bytes, ql[128]
// (low nibbles), qh[64] (2-bit highs), 16 int8 scales, fp16 d at 208.  Unit
// u is weights 64·(u%4) .. +63 of super-block u/4: half h = (u%4)/2 and
// p = u%2; weight j of the unit has its low nibble in ql[64h + j] (high
// nibble when p = 1), its top bits at 2·(2p + j/32) in qh[32h + j%32], and
// scale s[8h + 4p + j/16]; q = (low | top << 4) − 32.
struct Q6K {
  static constexpr uint32_t kFormat = 14;
  static constexpr uint32_t kUnit = 64;
  using Frag = Frag64;
  template <bool NORM>
  __device__ __forceinline__ static void load(const float *x, const float *nw, uint32_t u, Frag &f) {
    frag64_load<NORM>(x, nw, u, f);
  }
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) { frag64_from_lds(p, f); }
  struct Raw {
    uint32_t ql[16], qh[8], sc, d;
  };
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) {
    Raw r;
    const uint8_t *blk = row + (uint64_t)(u >> 2) * 210;
    const uint32_t h = (u >> 1) & 1, p = u & 1;
    load_dwords<16>(blk + 64 * h, r.ql);
    load_dwords<8>(blk + 128 + 32 * h, r.qh);
    load_dwords<1>(blk + 192 + 8 * h + 4 * p, &r.sc);
    // d: two bytes inside one aligned dword.
    const uintptr_t da = reinterpret_cast<uintptr_t>(blk + 208);
    r.d = *reinterpret_cast<const uint32_t *>(da & ~uintptr_t(3)) >> (8 * (da & 3));
    return r;
  }
  __device__ __forceinline__ static float compute(const Raw &r, uint32_t u, const Frag &f) {
    const uint32_t p = u & 1;
    float tot = 0.f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int i = 4 * g + k;  // dword of ql: weights 4i .. 4i+3
        const uint32_t lo = p ? (r.ql[i] >> 4) & 0x0f0f0f0fu : r.ql[i] & 0x0f0f0f0fu;
        const uint32_t top = (r.qh[i & 7] >> (2 * (2 * p + (i >> 3)))) & 0x03030303u;
        const uint32_t q = lo | (top << 4);
        if (k & 1)
          s1 = dot4u(q, f.x + 4 * i, s1);
        else
          s0 = dot4u(q, f.x + 4 * i, s0);
      }
      const float sc = (float)(int8_t)((r.sc >> (8 * g)) & 0xffu);
      tot = fmaf(sc, (s0 + s1) - 32.f * f.gs[g], tot);
    }
    return half_bits_to_float(r.d & 0xffffu) * tot;
  }
  __device__ __forceinline__ static float dot(const uint8_t *__restrict__ row, uint32_t u, const Frag &f) {
    return compute(fetch(row, u), u, f);
  }
};

// Q5_K (scalar.rs:157-176): 176-byte super-blocks of fp16 d and dmin, the
// 12 scale bytes of Q4_K, qh[32] (bit j of byte l is the fifth bit of
// element 32j + l) and qs[128] as Q4_K's nibbles.  A unit is the pair of
// 32-element blocks 2p, 2p+1 (the layout of the Q4K unit plus qh).
struct Q5K {
  static constexpr uint32_t kFormat = 13;
  static constexpr uint32_t kUnit = 64;
  using Frag = Q4K::Frag;
  template <bool NORM>
  __device__ __forceinline__ static void load(const float *x, const float *nw, uint32_t u, Frag &f) {
    Q4K::load<NORM>(x, nw, u, f);
  }
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) { Q4K::from_lds(p, f); }
  struct Raw {
    uint4 h, qh0, qh1, q0, q1;
  };
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) {
    const uint8_t *blk = row + (uint64_t)(u >> 2) * 176;
    const uint4 *hp = reinterpret_cast<const uint4 *>(blk);
    const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 48 + 32 * (u & 3));
    return Raw{hp[0], hp[1], hp[2], qp[0], qp[1]};
  }
  __device__ __forceinline__ static float compute(const Raw &raw, uint32_t u, const Frag &f) {
    const int p = u & 3;
    const uint32_t qw[8] = {raw.q0.x, raw.q0.y, raw.q0.z, raw.q0.w, raw.q1.x, raw.q1.y, raw.q1.z, raw.q1.w};
    const uint32_t hw[8] = {raw.qh0.x, raw.qh0.y, raw.qh0.z, raw.qh0.w, raw.qh1.x, raw.qh1.y, raw.qh1.z, raw.qh1.w};
    float s_lo0 = 0.f, s_lo1 = 0.f, s_hi0 = 0.f, s_hi1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t lo = (qw[k] & 0x0f0f0f0fu) | (((hw[k] >> (2 * p)) & 0x01010101u) << 4);
      const uint32_t hi = ((qw[k] >> 4) & 0x0f0f0f0fu) | (((hw[k] >> (2 * p + 1)) & 0x01010101u) << 4);
      s_lo0 = fmaf(ubyte0(lo), f.lo[4 * k + 0], s_lo0);
      s_lo1 = fmaf(ubyte1(lo), f.lo[4 * k + 1], s_lo1);
      s_lo0 = fmaf(ubyte2(lo), f.lo[4 * k + 2], s_lo0);
      s_lo1 = fmaf(ubyte3(lo), f.lo[4 * k + 3], s_lo1);
      s_hi0 = fmaf(ubyte0(hi), f.hi[4 * k + 0], s_hi0);
      s_hi1 = fmaf(ubyte1(hi), f.hi[4 * k + 1], s_hi1);
      s_hi0 = fmaf(ubyte2(hi), f.hi[4 * k + 2], s_hi0);
      s_hi1 = fmaf(ubyte3(hi), f.hi[4 * k + 3], s_hi1);
    }
    const uint32_t sc = q4k_pair_scales(raw.h.y, raw.h.z, raw.h.w, p);
    const float d = half_bits_to_float(raw.h.x & 0xffffu);
    const float dmin = half_bits_to_float(raw.h.x >> 16);
    const float qs = ubyte0(sc) * (s_lo0 + s_lo1) + ubyte1(sc) * (s_hi0 + s_hi1);
    const float ms = ubyte2(sc) * f.sum_lo + ubyte3(sc) * f.sum_hi;
    return d * qs - dmin * ms;
  }
  __device__ __forceinline__ static float dot(const uint8_t *__restrict__ row, uint32_t u, const Frag &f) {
    return compute(fetch(row, u), u, f);
  }
};

// --- Q4_K with integer activations --------------------------------------
//
// The decode GEMV's Q4_K path.  The staged input is quantised, once per
// workgroup, to 22-bit fixed point per 32-element block: with E the exponent
// of the block's largest |x| (|x| < 2^E), x_int = rint(x · 2^(21−E)), so
// every input carries an absolute error of at most 2^(E−22) — eight times
// the half-ulp 2^(E−25) of the block's largest element, and an element 2^-k
// times that largest one keeps about 22−k significant bits (the reference
// multiplies the f32 inputs themselves, quant.metal:364-386).  The error of a
// row is thus at most Σ_blocks Σ|w|·2^(E_b−22), far inside the reference's
// bound of 1e-5 of the row's Σ|w·x| (metal_matvec.rs:16-19).  x_int splits
// into three signed bytes x_int = d0 + 2^8·d1 + 2^16·d2 (d0, d1 in
// [−128, 127], d2 in [−32, 32]).  Then Σ q·x_int over a block is three
// v_dot4_i32_i8 per four nibbles on the raw nibble bytes, exact in int32
// (|Σ| ≤ 32·15·2^21 < 2^31), instead of a conversion and an FMA per weight;
// the block's scale 2^(E−21) is folded into the (d·sc) multiply.  The
// minimum term uses the block sums of the unquantised inputs.
constexpr uint32_t kDigitUnitBytes = 208;  // 3 planes × 2 blocks × 32 bytes, then xs[2], sum[2]

struct Q4K8 {
  static constexpr uint32_t kFormat = 12;
  static constexpr uint32_t kUnit = 64;
  static constexpr bool kDigits = true;
  struct Frag {
    uint32_t d[3][2][8];  // [digit][block of the pair][4 elements each]
    float xs[2], sum[2];
  };
  // The unit's digits and block constants from its slot in LDS.
  __device__ __forceinline__ static void from_lds(const float *p, Frag &f) {
    const uint4 *p4 = reinterpret_cast<const uint4 *>(p);
#pragma unroll
    for (int dg = 0; dg < 3; dg++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint4 a = p4[(dg * 2 + h) * 2], b = p4[(dg * 2 + h) * 2 + 1];
        f.d[dg][h][0] = a.x, f.d[dg][h][1] = a.y, f.d[dg][h][2] = a.z, f.d[dg][h][3] = a.w;
        f.d[dg][h][4] = b.x, f.d[dg][h][5] = b.y, f.d[dg][h][6] = b.z, f.d[dg][h][7] = b.w;
      }
    const float4 m = reinterpret_cast<const float4 *>(p)[12];
    f.xs[0] = m.x, f.xs[1] = m.y, f.sum[0] = m.z, f.sum[1] = m.w;
  }
  using Raw = Q4K::Raw;
  __device__ __forceinline__ static Raw fetch(const uint8_t *__restrict__ row, uint32_t u) { return Q4K::fetch(row, u); }
  __device__ __forceinline__ static float compute(const Raw &raw, uint32_t u, const Frag &f) {
    const int p = u & 3;
    const uint4 q0 = raw.q0, q1 = raw.q1;
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int lo = (int)(qw[k] & 0x0f0f0f0fu), hi = (int)((qw[k] >> 4) & 0x0f0f0f0fu);
      a0 = __builtin_amdgcn_sdot4(lo, (int)f.d[0][0][k], a0, false);
      a1 = __builtin_amdgcn_sdot4(lo, (int)f.d[1][0][k], a1, false);
      a2 = __builtin_amdgcn_sdot4(lo, (int)f.d[2][0][k], a2, false);
      b0 = __builtin_amdgcn_sdot4(hi, (int)f.d[0][1][k], b0, false);
      b1 = __builtin_amdgcn_sdot4(hi, (int)f.d[1][1][k], b1, false);
      b2 = __builtin_amdgcn_sdot4(hi, (int)f.d[2][1][k], b2, false);
    }
    const float v_lo = (float)(a0 + a1 * 256 + a2 * 65536);
    const float v_hi = (float)(b0 + b1 * 256 + b2 * 65536);
    const uint4 h = raw.h;
    const uint32_t sc = q4k_pair_scales(h.y, h.z, h.w, p);
    const float d = half_bits_to_float(h.x & 0xffffu);
    const float dmin = half_bits_to_float(h.x >> 16);
    const float qs = ubyte0(sc) * (f.xs[0] * v_lo) + ubyte1(sc) * (f.xs[1] * v_hi);
    const float ms = ubyte2(sc) * f.sum[0] + ubyte3(sc) * f.sum[1];
    return d * qs - dmin * ms;
  }
};

// Convert the staged inputs of a workgroup (n_units slots of kSlot floats,
// unit u's 64 inputs at slot u) into Q4K8's digit form, in place.  T
// threads; thread t takes chunks of 8 inputs c = t, t + T, ... (chunk c is
// inputs 8·(c % 8) .. +7 of unit c / 8); the four chunks of a 32-element
// block sit in four consecutive lanes of one wave.  Reads everything, waits
// for the whole workgroup, then writes.
template <int T, int kSlot, int kMaxChunks>
__device__ __forceinline__ void digitize_units(float *xs, uint32_t n_units) {
  const uint32_t tid = threadIdx.x, n_chunks = n_units * 8;
  float v[kMaxChunks][8];
#pragma unroll
  for (int i = 0; i < kMaxChunks; i++) {
    const uint32_t c = tid + (uint32_t)i * T;
    if (c < n_chunks) {
      const float4 *src = reinterpret_cast<const float4 *>(xs + (c / 8) * kSlot + (c % 8) * 8);
      const float4 a = src[0], b = src[1];
      v[i][0] = a.x, v[i][1] = a.y, v[i][2] = a.z, v[i][3] = a.w;
      v[i][4] = b.x, v[i][5] = b.y, v[i][6] = b.z, v[i][7] = b.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) v[i][j] = 0.f;
    }
  }
  uint32_t planes[kMaxChunks][3][2];
  float inv[kMaxChunks], sums[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; i++) {
    float mx = 0.f, sm = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      mx = fmaxf(mx, fabsf(v[i][j]));
      sm += v[i][j];
    }
    // The block's four chunks: consecutive lanes (T and the chunk numbering
    // keep c % 4 == lane % 4).
    // (DPP quad permutes: no LDS round trip; every lane runs this code.)
    mx = fmaxf(mx, dpp<kDppXor1>(mx));
    mx = fmaxf(mx, dpp<kDppXor2>(mx));
    sm += dpp<kDppXor1>(sm);
    sm += dpp<kDppXor2>(sm);
    int e = 0;
    if (mx > 0.f) frexpf(mx, &e);  // mx < 2^e
    const float scale = ldexpf(1.0f, 21 - e);
    inv[i] = ldexpf(1.0f, e - 21);
    sums[i] = sm;
    uint32_t pk[3][2] = {};
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int xi = (int)rintf(v[i][j] * scale);
      const int d0 = (int)(int8_t)(xi & 0xff);
      const int r = (xi - d0) >> 8;
      const int d1 = (int)(int8_t)(r & 0xff);
      const int d2 = (r - d1) >> 8;
      const int sh = 8 * (j % 4);
      pk[0][j / 4] |= ((uint32_t)d0 & 0xffu) << sh;
      pk[1][j / 4] |= ((uint32_t)d1 & 0xffu) << sh;
      pk[2][j / 4] |= ((uint32_t)d2 & 0xffu) << sh;
    }
#pragma unroll
    for (int dg = 0; dg < 3; dg++) planes[i][dg][0] = pk[dg][0], planes[i][dg][1] = pk[dg][1];
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < kMaxChunks; i++) {
    const uint32_t c = tid + (uint32_t)i * T;
    if (c < n_chunks) {
      uint8_t *slot = reinterpret_cast<uint8_t *>(xs + (c / 8) * kSlot);
      const uint32_t h = (c % 8) / 4, j0 = (c % 4) * 8;
#pragma unroll
      for (int dg = 0; dg < 3; dg++)
        *reinterpret_cast<uint2 *>(slot + (dg * 2 + h) * 32 + j0) = make_uint2(planes[i][dg][0], planes[i][dg][1]);
      if (c % 4 == 0) {
        reinterpret_cast<float *>(slot + 192)[h] = inv[i];
        reinterpret_cast<float *>(slot + 200)[h] = sums[i];
      }
    }
  }
}

}  // namespace bch
