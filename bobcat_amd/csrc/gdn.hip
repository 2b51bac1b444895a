// Gated DeltaNet kernels and the output gate of Qwen3.5's attention: the
// MI355X counterparts of gdn_conv / gdn_gates / gdn_recurrence /
// gdn_gated_norm / attention_gate (crates/bobcat-metal/src/gdn.metal) and of
// the CPU Model::delta_net (crates/bobcat/src/qwen35.rs:430-516).
//
// The recurrence gives every column of a value head's state its own wave:
// a column evolves on its own given the token's key, query, value entry and
// gates (remembered_c = Σ_r S[r][c]·k[r], S[r][c] += k[r]·β(v_c − remembered_c),
// out_c = Σ_r S[r][c]·q[r]), so the k_dim rows of a column live in the
// registers of one wave (k_dim/64 per lane) for a whole prefill batch and the
// two dot products per token are wave reductions.  16 heads of 128 columns
// make 2048 waves.  The workgroup stages 32 tokens at a time in LDS (the
// normalised query and key, its columns' values, the gates), so the
// sequential token loop reads LDS instead of waiting on memory per token.
#include <cmath>

#include "device.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr int kGdnCols = 4;  // columns (waves) per workgroup

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
// transformers' softplus returns its input above 20 (qwen35.rs:775-778).
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

constexpr int kGdnChunk = 32;  // tokens staged in LDS at a time

template <int RPL>
__global__ __launch_bounds__(kGdnCols * 64) void k_gdn_recurrence(GdnArgs a) {
  constexpr int KD = RPL * 64;  // k_dim
  // A chunk of tokens staged by the workgroup: the l2-normalised query
  // (times q_scale) and key of this head, the four columns' values, and
  // the gates.  The token loop then waits on LDS, not on memory.
  __shared__ float qs[kGdnChunk][KD], ks[kGdnChunk][KD], vs[kGdnChunk][kGdnCols], bs[kGdnChunk], ds[kGdnChunk];
  const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const uint32_t col0 = blockIdx.x * kGdnCols, col = col0 + wave, head = blockIdx.y;
  const uint32_t key_head = head % a.n_k, key_dim = a.n_k * a.k_dim, conv_dim = 2 * key_dim + a.n_v * a.v_dim;
  const uint32_t r0 = lane * RPL;
  float *S = a.state + (uint64_t)head * a.k_dim * a.v_dim;
  float rows[RPL];
#pragma unroll
  for (int i = 0; i < RPL; i++) rows[i] = S[(uint64_t)(r0 + i) * a.v_dim + col];
  for (uint32_t t0 = 0; t0 < a.n_tokens; t0 += kGdnChunk) {
    const uint32_t n = min((uint32_t)kGdnChunk, a.n_tokens - t0);
    __syncthreads();  // the previous chunk is consumed
    // Wave w stages tokens w, w + 4, ...: l2_normalize of the query and the
    // key (qwen35.rs:464-470), each lane holding rows r0 .. r0+RPL-1.
    for (uint32_t j = wave; j < n; j += kGdnCols) {
      const float *tok = a.y + (uint64_t)(t0 + j) * conv_dim;
      float q[RPL], k[RPL], sq = 0.f, sk = 0.f;
#pragma unroll
      for (int i = 0; i < RPL; i++) {
        q[i] = tok[key_head * a.k_dim + r0 + i];
        k[i] = tok[key_dim + key_head * a.k_dim + r0 + i];
      }
#pragma unroll
      for (int i = 0; i < RPL; i++) {
        sq = fmaf(q[i], q[i], sq);
        sk = fmaf(k[i], k[i], sk);
      }
      sq = wave_sum(sq);
      sk = wave_sum(sk);
      const float fq = a.q_scale / sqrtf(sq + 1e-6f), fk = 1.0f / sqrtf(sk + 1e-6f);
#pragma unroll
      for (int i = 0; i < RPL; i++) {
        qs[j][r0 + i] = q[i] * fq;
        ks[j][r0 + i] = k[i] * fk;
      }
      if (lane < kGdnCols) vs[j][lane] = tok[2 * key_dim + head * a.v_dim + col0 + lane];
      if (lane == 0) {
        const uint64_t gs = a.gate_stride ? a.gate_stride : a.n_v;
        const float b = a.beta[(uint64_t)(t0 + j) * gs + head];
        const float d = a.alpha[(uint64_t)(t0 + j) * gs + head];
        bs[j] = a.raw_gates ? sigmoid_f(b) : b;
        ds[j] = a.raw_gates ? expf(a.a[head] * softplus_f(d + a.dt_bias[head])) : d;
      }
    }
    __syncthreads();
    for (uint32_t j = 0; j < n; j++) {
      const float decay = ds[j], beta = bs[j];
      float rem = 0.f;
#pragma unroll
      for (int i = 0; i < RPL; i++) {
        rows[i] *= decay;
        rem = fmaf(rows[i], ks[j][r0 + i], rem);
      }
      rem = wave_sum(rem);
      const float delta = (vs[j][wave] - rem) * beta;
      float o = 0.f;
#pragma unroll
      for (int i = 0; i < RPL; i++) {
        rows[i] = fmaf(ks[j][r0 + i], delta, rows[i]);
        o = fmaf(rows[i], qs[j][r0 + i], o);
      }
      o = wave_sum(o);
      if (lane == 0) a.out[(uint64_t)(t0 + j) * a.n_v * a.v_dim + head * a.v_dim + col] = o;
    }
  }
#pragma unroll
  for (int i = 0; i < RPL; i++) S[(uint64_t)(r0 + i) * a.v_dim + col] = rows[i];
}

// One token (decode): a workgroup per value head, CB blocks of 64 columns;
// in block cb lane c owns column 64·cb + c of the head's state and wave w of
// the block rows [w·KD/4, (w+1)·KD/4), so each row of a block is one
// coalesced 256-byte access; the two dot products over the rows are per-lane
// sums, then a sum over the block's four waves in LDS (in wave order).  (The
// wave-per-column form above spreads a column over 64 lanes, which touches a
// cache line per row and per column.)  With norm_w the head's output gets
// the gated norm of k_gdn_gated_norm in the same workgroup.
template <int KD, int CB>
__global__ __launch_bounds__(256 * CB) void k_gdn_step(GdnArgs a) {
  constexpr int RW = KD / 4;  // rows per wave
  __shared__ float qn[KD], kn[KD], part[CB][4][64];
  __shared__ float gate_s[2], ss_s[CB];
  const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const uint32_t cb = wave / 4, wq = wave % 4;
  const uint32_t head = blockIdx.y, col = cb * 64 + lane;
  const uint32_t key_head = head % a.n_k, key_dim = a.n_k * a.k_dim;
  const float *tok = a.y;
  float *S = a.state + (uint64_t)head * KD * a.v_dim + col;
  // The token's small inputs first, then the state rows: memory returns in
  // issue order, so the norms below wait for the small loads alone and run
  // while the state streams in.  The loads are unconditional (every wave
  // reads a query or key row; waves past 1 discard theirs), so the waits
  // count exactly.
  const float *src = tok + (wave == 1 ? key_dim : 0u) + key_head * KD;
  float e[KD / 64];
#pragma unroll
  for (int i = 0; i < KD / 64; i++) e[i] = src[lane * (KD / 64) + i];
  const float v = tok[2 * key_dim + head * a.v_dim + col];
  const float gz = a.norm_w ? a.gate_z[(uint64_t)head * a.v_dim + col] : 0.f;
  const float nw = a.norm_w ? a.norm_w[col] : 0.f;
  // The head's gate inputs (uniform: scalar loads).
  const float gb = a.beta[head], gd = a.alpha[head];
  const float ga = a.raw_gates ? a.a[head] : 0.f, gdt = a.raw_gates ? a.dt_bias[head] : 0.f;
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  float rows[RW];
#pragma unroll
  for (int i = 0; i < RW; i++) rows[i] = S[(uint64_t)(wq * RW + i) * a.v_dim];
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // Waves 0 and 1 normalise the query and the key (qwen35.rs:464-470).
  if (wave < 2) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < KD / 64; i++) ss = fmaf(e[i], e[i], ss);
    ss = wave_sum(ss);
    const float f = wave == 0 ? a.q_scale / sqrtf(ss + 1e-6f) : 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
    for (int i = 0; i < KD / 64; i++) (wave == 0 ? qn : kn)[lane * (KD / 64) + i] = e[i] * f;
  } else if (wave == 2 && lane == 0) {
    gate_s[0] = a.raw_gates ? sigmoid_f(gb) : gb;
    gate_s[1] = a.raw_gates ? expf(ga * softplus_f(gd + gdt)) : gd;
  }
  __syncthreads();
  const float beta = gate_s[0], decay = gate_s[1];
  float rem = 0.f;
#pragma unroll
  for (int i = 0; i < RW; i++) {
    rows[i] *= decay;
    rem = fmaf(rows[i], kn[wq * RW + i], rem);
  }
  part[cb][wq][lane] = rem;
  __syncthreads();
  rem = (part[cb][0][lane] + part[cb][1][lane]) + (part[cb][2][lane] + part[cb][3][lane]);
  const float delta = (v - rem) * beta;
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < RW; i++) {
    rows[i] = fmaf(kn[wq * RW + i], delta, rows[i]);
    o = fmaf(rows[i], qn[wq * RW + i], o);
    S[(uint64_t)(wq * RW + i) * a.v_dim] = rows[i];
  }
  __syncthreads();
  part[cb][wq][lane] = o;
  __syncthreads();
  o = (part[cb][0][lane] + part[cb][1][lane]) + (part[cb][2][lane] + part[cb][3][lane]);
  float *orow = a.out + (uint64_t)head * a.v_dim;
  if (!a.norm_w) {
    if (wq == 0) orow[col] = o;
    return;
  }
  // The gated norm of the head: RMS over its v_dim outputs (block sums in
  // block order), then w ⊙ (o·scale) ⊙ silu(z).
  if (wq == 0) {
    const float ss = wave_sum(o * o);
    if (lane == 0) ss_s[cb] = ss;
  }
  __syncthreads();
  if (wq != 0) return;
  float ss = 0.f;
#pragma unroll
  for (int b = 0; b < CB; b++) ss += ss_s[b];
  const float scale = rsqrtf(ss / (float)a.v_dim + a.norm_eps);
  orow[col] = nw * (o * scale) * (gz / (1.0f + expf(-gz)));
}

bool gdn_step_supported(const GdnArgs &a) {
  return a.n_tokens == 1 && a.v_dim % kGdnCols == 0 && a.v_dim % 64 == 0 && a.v_dim <= 256 &&
         (a.k_dim == 64 || a.k_dim == 128);
}

bool run_gdn_recurrence(hipStream_t s, const GdnArgs &a) {
  if (a.v_dim % kGdnCols || a.n_tokens == 0) return false;
  if (gdn_step_supported(a)) {
    const uint32_t cb = a.v_dim / 64;
    const dim3 grid(1, a.n_v);
#define BCH_STEP(KD, CB) k_gdn_step<KD, CB><<<grid, 256 * CB, 0, s>>>(a)
    if (a.k_dim == 64) {
      if (cb == 1) BCH_STEP(64, 1); else if (cb == 2) BCH_STEP(64, 2); else if (cb == 3) BCH_STEP(64, 3); else BCH_STEP(64, 4);
    } else {
      if (cb == 1) BCH_STEP(128, 1); else if (cb == 2) BCH_STEP(128, 2); else if (cb == 3) BCH_STEP(128, 3); else BCH_STEP(128, 4);
    }
#undef BCH_STEP
    return true;
  }
  const dim3 grid(a.v_dim / kGdnCols, a.n_v);
  if (a.k_dim == 64)
    k_gdn_recurrence<1><<<grid, kGdnCols * 64, 0, s>>>(a);
  else if (a.k_dim == 128)
    k_gdn_recurrence<2><<<grid, kGdnCols * 64, 0, s>>>(a);
  else
    return false;
  return true;
}

// --- chunked prefill ------------------------------------------------------
//
// The gated delta rule over a chunk of C tokens from the state S0 at its
// start, with gamma_t the product of the decays up to token t (from the
// chunk's start), reads (the WY/UT form of the delta rule):
//   A[t][s] = beta_t (gamma_t / gamma_s) k_t.k_s          s < t
//   (I + A) D = diag(beta) (V - diag(gamma) K S0)         D = the chunk's deltas
//   D = U - W S0,  U = (I + A)^-1 diag(beta) V,  W = (I + A)^-1 diag(beta gamma) K
//   O = diag(gamma) Q S0 + P D,  P[t][s] = (gamma_t / gamma_s) q_t.k_s   s <= t
//   S_C = gamma_C S0 + Kt^T D,   Kt[s] = (gamma_C / gamma_s) k_s
// which unrolls the per-token recurrence of qwen35.rs:475-511 exactly (in
// exact arithmetic).  k_gdn_chunk_prep computes W, U, P, diag(gamma) Q, Kt
// and gamma_C for every (chunk, head) at once: U and W by forward
// substitution, one thread per column; the decays as differences of a
// float64 running sum of log-decays.  k_gdn_chunk_scan then carries the
// state through the chunks: each column of S evolves on its own, so a
// workgroup owns NC columns of one head and walks the chunks in order.

constexpr int kGdnC = 64;  // tokens per chunk

__host__ __device__ constexpr uint64_t gdn_chunk_floats(uint32_t kd, uint32_t vd) {
  return 64ull * (3ull * kd + vd) + 64ull * 64ull + 64ull;
}

template <int KD>
__global__ __launch_bounds__(256) void k_gdn_chunk_prep(GdnArgs a, float *__restrict__ scratch, uint32_t n_chunks) {
  constexpr int C = kGdnC, KP = KD + 1, R = KD / 64;
  __shared__ float qs[C][KP], ks[C][KP];
  __shared__ __align__(16) float amT[C][C + 4];  // A transposed: amT[u][t] = A[t][u]
  __shared__ float bs[C], wgam[C];
  __shared__ double lg[C];
  const uint32_t tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const uint32_t chunk = blockIdx.x, head = blockIdx.y;
  const uint32_t vd = a.v_dim;
  const uint32_t t0 = chunk * C, L = min((uint32_t)C, a.n_tokens - t0);
  const uint32_t key_head = head % a.n_k, key_dim = a.n_k * KD, conv_dim = 2 * key_dim + a.n_v * vd;
  float *base = scratch + ((uint64_t)head * n_chunks + chunk) * gdn_chunk_floats(KD, vd);
  float *Wg = base, *Ug = Wg + C * KD, *Qg = Ug + (uint64_t)C * vd, *Kt = Qg + C * KD, *Pg = Kt + C * KD;
  float *gC = Pg + C * C;
  // The value column this thread solves first (column tid of [W | U] when it
  // is a U column), loaded before anything else: nothing before the forward
  // substitution depends on it.
  const bool pre_u = tid >= (uint32_t)KD && tid < KD + vd;
  float vpre[C];
  {
    const float *v = a.y + (uint64_t)t0 * conv_dim + 2 * key_dim + head * vd + (pre_u ? tid - KD : 0);
#pragma unroll
    for (int t = 0; t < C; t++) vpre[t] = pre_u && (uint32_t)t < L ? v[(uint64_t)t * conv_dim] : 0.f;
  }
  // The l2-normalised query (times q_scale) and key of each token
  // (qwen35.rs:464-470); rows past the chunk's end are zero.  Wave w takes
  // tokens w, w+4, ..., all of their loads issued before any is used.
  {
    constexpr int TW = C / 4;  // tokens per wave
    float q[TW][R], k[TW][R];
#pragma unroll
    for (int jj = 0; jj < TW; jj++) {
      const uint32_t j = wave + 4 * jj;
      const float *tok = a.y + (uint64_t)(t0 + min(j, L - 1)) * conv_dim;
#pragma unroll
      for (int i = 0; i < R; i++) {
        q[jj][i] = j < L ? tok[key_head * KD + lane * R + i] : 0.f;
        k[jj][i] = j < L ? tok[key_dim + key_head * KD + lane * R + i] : 0.f;
      }
    }
#pragma unroll
    for (int jj = 0; jj < TW; jj++) {
      const uint32_t j = wave + 4 * jj;
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int i = 0; i < R; i++) {
        sq = fmaf(q[jj][i], q[jj][i], sq);
        sk = fmaf(k[jj][i], k[jj][i], sk);
      }
      sq = wave_sum(sq);
      sk = wave_sum(sk);
      const float fq = a.q_scale / sqrtf(sq + 1e-6f), fk = 1.0f / sqrtf(sk + 1e-6f);
#pragma unroll
      for (int i = 0; i < R; i++) {
        qs[j][lane * R + i] = q[jj][i] * fq;
        ks[j][lane * R + i] = k[jj][i] * fk;
      }
    }
  }
  // Gates: beta, and the running sum of the log-decays in float64.
  if (wave == 0) {
    float b = 0.f, l = 0.f;
    if (lane < L) {
      const uint64_t gs = a.gate_stride ? a.gate_stride : a.n_v;
      const float rb = a.beta[(uint64_t)(t0 + lane) * gs + head];
      const float rd = a.alpha[(uint64_t)(t0 + lane) * gs + head];
      b = a.raw_gates ? sigmoid_f(rb) : rb;
      l = a.raw_gates ? a.a[head] * softplus_f(rd + a.dt_bias[head]) : logf(rd);
    }
    double v = l;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double o = __shfl_up(v, off, 64);
      if (lane >= (uint32_t)off) v += o;
    }
    bs[lane] = b;
    lg[lane] = v;
    wgam[lane] = lane < L ? b * expf((float)v) : 0.f;
  }
  __syncthreads();
  const double lC = lg[L - 1];
  // A (strictly lower) and P (lower with the diagonal): 4x4 blocks per thread.
  {
    const uint32_t ti = tid / 16, si = tid % 16;
    float kk[4][4] = {}, qk[4][4] = {};
    for (int r = 0; r < KD; r++) {
      float kt[4], qt[4], kv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        kt[i] = ks[4 * ti + i][r];
        qt[i] = qs[4 * ti + i][r];
        kv[i] = ks[4 * si + i][r];
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          kk[i][j] = fmaf(kt[i], kv[j], kk[i][j]);
          qk[i][j] = fmaf(qt[i], kv[j], qk[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t t = 4 * ti + i, u = 4 * si + j;
        const float dec = (u <= t && t < L) ? expf((float)(lg[t] - lg[u])) : 0.f;
        amT[u][t] = u < t ? bs[t] * dec * kk[i][j] : 0.f;
        Pg[t * C + u] = dec * qk[i][j];
      }
  }
  // diag(gamma) Q and Kt, and gamma_C.
  for (uint32_t e = tid; e < (uint32_t)(C * KD); e += 256) {
    const uint32_t t = e / KD, r = e % KD;
    const float gt = t < L ? expf((float)lg[t]) : 0.f;
    const float kc = t < L ? expf((float)(lC - lg[t])) : 0.f;
    Qg[e] = gt * qs[t][r];
    Kt[e] = kc * ks[t][r];
  }
  if (tid == 0) gC[0] = expf((float)lC);
  __syncthreads();
  // W and U by forward substitution, x_t = rhs_t - sum_{s<t} A[t][s] x_s,
  // one thread per column of [W | U].
  for (uint32_t col = tid; col < KD + vd; col += 256) {
    float x[C];
    if (col < KD) {
#pragma unroll
      for (int t = 0; t < C; t++) x[t] = wgam[t] * ks[t][col];
    } else if (col == tid) {
#pragma unroll
      for (int t = 0; t < C; t++) x[t] = (uint32_t)t < L ? bs[t] * vpre[t] : 0.f;
    } else {
      const float *v = a.y + (uint64_t)t0 * conv_dim + 2 * key_dim + head * vd + (col - KD);
#pragma unroll
      for (int t = 0; t < C; t++) x[t] = (uint32_t)t < L ? bs[t] * v[(uint64_t)t * conv_dim] : 0.f;
    }
    // Column by column: once x_u is final it enters every later row, so
    // each step has up to 63 independent FMAs (a row-by-row loop waits on
    // one dependent chain of 2016).  Every row still adds its terms in
    // order u = 0, 1, ..., as the row-by-row form does.
#pragma unroll
    for (int u = 0; u < C - 1; u++) {
      // Rows u+1 .. C-1 of column u, four per 16-byte LDS read.
#pragma unroll
      for (int t4 = (u + 1) / 4; t4 < C / 4; t4++) {
        const float4 a4 = *reinterpret_cast<const float4 *>(&amT[u][4 * t4]);
        const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (4 * t4 + i > u) x[4 * t4 + i] = fmaf(-av[i], x[u], x[4 * t4 + i]);
      }
    }
    if (col < KD) {
#pragma unroll
      for (int t = 0; t < C; t++) Wg[t * KD + col] = x[t];
    } else {
#pragma unroll
      for (int t = 0; t < C; t++) Ug[(uint64_t)t * vd + (col - KD)] = x[t];
    }
  }
}

template <int KD, int NC>
__global__ __launch_bounds__(256) void k_gdn_chunk_scan(GdnArgs a, const float *__restrict__ scratch,
                                                        uint32_t n_chunks) {
  constexpr int C = kGdnC, KP = KD + 4;
  static_assert(NC == 8, "the thread layout below assumes 8 columns");
  __shared__ __align__(16) float w_s[C][KP], q_s[C][KP], k_s[C][KP];
  __shared__ float p_s[C][C + 1];
  __shared__ __align__(16) float s_s[KD][NC], d_s[C][NC];
  const uint32_t tid = threadIdx.x, vd = a.v_dim;
  // Blocks are numbered so that the column blocks of one head run on one
  // XCD (workgroup i goes to XCD i % 8) and share its L2.
  const uint32_t n_cb = vd / NC, total = n_cb * a.n_v;
  uint32_t v = blockIdx.x;
  if (total % 8 == 0) v = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
  const uint32_t head = v / n_cb, col0 = (v % n_cb) * NC;
  float *S = a.state + (uint64_t)head * KD * vd + col0;
  // This thread's state entries: row r = tid / 2, columns c0 .. c0 + 3.
  const uint32_t sr = tid / 2, sc = (tid % 2) * 4;
  float srow[4];
  if (sr < (uint32_t)KD) {
#pragma unroll
    for (int j = 0; j < 4; j++) srow[j] = s_s[sr][sc + j] = S[(uint64_t)sr * vd + sc + j];
  }
  // Delta / output entries: token t = tid / 4, columns dc, dc + 1.
  const uint32_t dt = tid / 4, dc = (tid % 4) * 2;
  for (uint32_t c = 0; c < n_chunks; c++) {
    const float *base = scratch + ((uint64_t)head * n_chunks + c) * gdn_chunk_floats(KD, vd);
    const float *Wg = base, *Ug = Wg + C * KD, *Qg = Ug + (uint64_t)C * vd, *Kt = Qg + C * KD, *Pg = Kt + C * KD;
    const float gC = Pg[C * C];
    const uint32_t t0 = c * C, L = min((uint32_t)C, a.n_tokens - t0);
    // Stage W, diag(gamma) Q, Kt and P.
    for (uint32_t e = tid; e < (uint32_t)(C * KD / 4); e += 256) {
      const uint32_t t = e / (KD / 4), r4 = e % (KD / 4);
      const float4 w = reinterpret_cast<const float4 *>(Wg)[e];
      const float4 q = reinterpret_cast<const float4 *>(Qg)[e];
      const float4 k = reinterpret_cast<const float4 *>(Kt)[e];
      *reinterpret_cast<float4 *>(&w_s[t][4 * r4]) = w;
      *reinterpret_cast<float4 *>(&q_s[t][4 * r4]) = q;
      *reinterpret_cast<float4 *>(&k_s[t][4 * r4]) = k;
    }
    for (uint32_t e = tid; e < (uint32_t)(C * C); e += 256) p_s[e / C][e % C] = Pg[e];
    const float u0 = Ug[(uint64_t)dt * vd + col0 + dc], u1 = Ug[(uint64_t)dt * vd + col0 + dc + 1];
    __syncthreads();
    // D = U - W S0 (16- and 8-byte LDS reads; r ascending as before).
    float d0 = u0, d1 = u1;
    for (int r = 0; r < KD; r += 4) {
      const float4 w4 = *reinterpret_cast<const float4 *>(&w_s[dt][r]);
      const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float2 s2 = *reinterpret_cast<const float2 *>(&s_s[r + i][dc]);
        d0 = fmaf(-wv[i], s2.x, d0);
        d1 = fmaf(-wv[i], s2.y, d1);
      }
    }
    d_s[dt][dc] = d0;
    d_s[dt][dc + 1] = d1;
    __syncthreads();
    // O = diag(gamma) Q S0 + P D.
    float o0 = 0.f, o1 = 0.f;
    for (int r = 0; r < KD; r += 4) {
      const float4 q4 = *reinterpret_cast<const float4 *>(&q_s[dt][r]);
      const float qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float2 s2 = *reinterpret_cast<const float2 *>(&s_s[r + i][dc]);
        o0 = fmaf(qv[i], s2.x, o0);
        o1 = fmaf(qv[i], s2.y, o1);
      }
    }
    for (uint32_t u = 0; u <= dt; u++) {
      const float pv = p_s[dt][u];
      const float2 d2 = *reinterpret_cast<const float2 *>(&d_s[u][dc]);
      o0 = fmaf(pv, d2.x, o0);
      o1 = fmaf(pv, d2.y, o1);
    }
    if (dt < L) {
      float *orow = a.out + (uint64_t)(t0 + dt) * a.n_v * vd + head * vd + col0;
      orow[dc] = o0;
      orow[dc + 1] = o1;
    }
    // S_C = gamma_C S0 + Kt^T D.
    if (sr < (uint32_t)KD) {
      float acc[4];
#pragma unroll
      for (int j = 0; j < 4; j++) acc[j] = gC * srow[j];
      for (int u = 0; u < C; u++) {
        const float kv = k_s[u][sr];
        const float4 d4 = *reinterpret_cast<const float4 *>(&d_s[u][sc]);
        acc[0] = fmaf(kv, d4.x, acc[0]);
        acc[1] = fmaf(kv, d4.y, acc[1]);
        acc[2] = fmaf(kv, d4.z, acc[2]);
        acc[3] = fmaf(kv, d4.w, acc[3]);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) srow[j] = acc[j];
    }
    __syncthreads();  // every read of s_s and of the staged chunk is done
    if (sr < (uint32_t)KD) {
#pragma unroll
      for (int j = 0; j < 4; j++) s_s[sr][sc + j] = srow[j];
    }
  }
  if (sr < (uint32_t)KD) {
#pragma unroll
    for (int j = 0; j < 4; j++) S[(uint64_t)sr * vd + sc + j] = srow[j];
  }
}

constexpr int kGdnScanCols = 8;

bool gdn_chunked_supported(const GdnArgs &a) {
  return (a.k_dim == 64 || a.k_dim == 128) && a.v_dim % kGdnScanCols == 0 && a.v_dim <= 256 && a.n_tokens > 0;
}

uint64_t gdn_chunk_scratch_floats(uint32_t n_v, uint32_t k_dim, uint32_t v_dim, uint32_t n_tokens) {
  const uint64_t chunks = (n_tokens + kGdnC - 1) / kGdnC;
  return (uint64_t)n_v * chunks * gdn_chunk_floats(k_dim, v_dim);
}

bool run_gdn_chunked(hipStream_t s, const GdnArgs &a, float *scratch) {
  if (!gdn_chunked_supported(a)) return false;
  const uint32_t n_chunks = (a.n_tokens + kGdnC - 1) / kGdnC;
  const dim3 prep(n_chunks, a.n_v);
  const uint32_t scan = a.n_v * (a.v_dim / kGdnScanCols);
  if (a.k_dim == 64) {
    k_gdn_chunk_prep<64><<<prep, 256, 0, s>>>(a, scratch, n_chunks);
    k_gdn_chunk_scan<64, kGdnScanCols><<<scan, 256, 0, s>>>(a, scratch, n_chunks);
  } else {
    k_gdn_chunk_prep<128><<<prep, 256, 0, s>>>(a, scratch, n_chunks);
    k_gdn_chunk_scan<128, kGdnScanCols><<<scan, 256, 0, s>>>(a, scratch, n_chunks);
  }
  return true;
}

// The causal convolution with SiLU of gdn_conv / the DeltaNet step
// (qwen35.rs:448-462), one thread per (token, channel): input t - past + i
// comes from the batch or, before it, from `hist`.  The newest term is added
// first, then the window oldest first, as the reference adds them.  A second
// launch then leaves the latest k-1 inputs in `hist` (after every read of
// the old history).
__global__ void k_gdn_conv(const float *__restrict__ x, const float *__restrict__ taps, const float *__restrict__ hist,
                           float *__restrict__ y, uint32_t channels, uint32_t ksize, uint32_t n_tokens,
                           uint32_t x_stride) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (uint64_t)n_tokens * channels) return;
  const uint32_t t = (uint32_t)(i / channels), c = (uint32_t)(i % channels), past = ksize - 1;
  const float *tp = taps + (uint64_t)c * ksize;
  float sum = tp[past] * x[(uint64_t)t * x_stride + c];
  for (uint32_t j = 0; j < past; j++) {
    const int src = (int)t - (int)past + (int)j;  // token of window slot j
    const float w = src >= 0 ? x[(uint64_t)src * x_stride + c] : hist[(uint64_t)c * past + (past + src)];
    sum += tp[j] * w;
  }
  y[i] = sum / (1.0f + expf(-sum));
}

__global__ void k_gdn_conv_history(const float *__restrict__ x, float *__restrict__ hist, uint32_t channels,
                                   uint32_t ksize, uint32_t n_tokens, uint32_t x_stride) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= channels) return;
  const uint32_t past = ksize - 1;
  float window[kGdnMaxKernel - 1];
  for (uint32_t j = 0; j < past; j++) {
    const int src = (int)n_tokens - (int)past + (int)j;
    window[j] = src >= 0 ? x[(uint64_t)src * x_stride + c] : hist[(uint64_t)c * past + (past + src)];
  }
  for (uint32_t j = 0; j < past; j++) hist[(uint64_t)c * past + j] = window[j];
}

void run_gdn_conv(hipStream_t s, const float *x, const float *taps, float *hist, float *y, uint32_t channels,
                  uint32_t ksize, uint32_t n_tokens, uint32_t x_stride) {
  const uint64_t n = (uint64_t)n_tokens * channels;
  if (!n) return;
  const uint32_t xs = x_stride ? x_stride : channels;
  k_gdn_conv<<<(uint32_t)((n + 255) / 256), 256, 0, s>>>(x, taps, hist, y, channels, ksize, n_tokens, xs);
  k_gdn_conv_history<<<(channels + 255) / 256, 256, 0, s>>>(x, hist, channels, ksize, n_tokens, xs);
}

// gdn_gates (gdn.metal:125-149): beta <- sigmoid(beta), alpha <- the decay
// exp(a·softplus(alpha + dt_bias)), per value head of each token.
__global__ void k_gdn_gates(float *beta, float *alpha, const float *a, const float *dt_bias, uint32_t n_v,
                            uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t h = i % n_v;
  beta[i] = sigmoid_f(beta[i]);
  alpha[i] = expf(a[h] * softplus_f(alpha[i] + dt_bias[h]));
}

void run_gdn_gates(hipStream_t s, float *beta, float *alpha, const float *a, const float *dt_bias, uint32_t n_v,
                   uint32_t n) {
  k_gdn_gates<<<(n + 255) / 256, 256, 0, s>>>(beta, alpha, a, dt_bias, n_v, n);
}

// The gated output norm (qwen35.rs:505-511): one wave per row of v_dim.
__global__ __launch_bounds__(64) void k_gdn_gated_norm(float *x, const float *__restrict__ w,
                                                       const float *__restrict__ z, uint32_t v_dim, float eps,
                                                       uint32_t n_v, uint32_t z_stride) {
  float *row = x + (uint64_t)blockIdx.x * v_dim;
  const float *g = z_stride ? z + (uint64_t)(blockIdx.x / n_v) * z_stride + (uint64_t)(blockIdx.x % n_v) * v_dim
                            : z + (uint64_t)blockIdx.x * v_dim;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < v_dim; i += 64) ss = fmaf(row[i], row[i], ss);
  ss = wave_sum(ss);
  const float scale = (float)(1.0 / sqrt((double)ss / (double)v_dim + (double)eps));
  for (uint32_t i = threadIdx.x; i < v_dim; i += 64) {
    const float gi = g[i];
    row[i] = w[i] * (row[i] * scale) * (gi / (1.0f + expf(-gi)));
  }
}

void run_gdn_gated_norm(hipStream_t s, float *x, const float *w, const float *z, uint32_t v_dim, uint32_t n_rows,
                        float eps, uint32_t n_v, uint32_t z_stride) {
  k_gdn_gated_norm<<<n_rows, 64, 0, s>>>(x, w, z, v_dim, eps, std::max(1u, n_v), z_stride);
}

// attention_gate (gdn.metal:306-322): each query head's output times the
// sigmoid of its gate, which follows its queries in the projection.
__global__ void k_attention_gate(float *attn, const float *q_gate, uint32_t head_dim, uint32_t q_dim, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t t = i / q_dim;
  const uint32_t e = (uint32_t)(i % q_dim), h = e / head_dim, d = e % head_dim;
  attn[i] *= sigmoid_f(q_gate[t * 2 * q_dim + (uint64_t)(2 * h + 1) * head_dim + d]);
}

void run_attention_gate(hipStream_t s, float *attn, const float *q_gate, uint32_t head_dim, uint32_t q_dim,
                        uint32_t n_tokens) {
  const uint64_t n = (uint64_t)n_tokens * q_dim;
  k_attention_gate<<<(uint32_t)((n + 255) / 256), 256, 0, s>>>(attn, q_gate, head_dim, q_dim, n);
}

}  // namespace bch

// ---------------------------------------------------------------------
// C ABI (Metal::gdn_conv / gdn_gates / gdn_recurrence / gdn_gated_norm /
// attention_gate, crates/bobcat-metal/src/backend.rs).
// ---------------------------------------------------------------------

using namespace bch;

extern "C" int bch_gdn_conv(bch_ctx *ctx, bch_view x, bch_view taps, bch_view history, bch_view y, uint32_t channels,
                            uint32_t kernel_size, uint32_t n_tokens) {
  if (kernel_size < 2 || kernel_size > kGdnMaxKernel)
    return fail(BCH_ERR_DELTANET_LIMITS, "gdn_conv: 2 to %u taps, got %u", kGdnMaxKernel, kernel_size);
  const float *xp, *tp;
  float *hp, *yp;
  BCH_TRY(view_ptr(ctx, "gdn_conv", x, (uint64_t)n_tokens * channels * 4, &xp));
  BCH_TRY(view_ptr(ctx, "gdn_conv", taps, (uint64_t)channels * kernel_size * 4, &tp));
  BCH_TRY(view_ptr(ctx, "gdn_conv", history, (uint64_t)channels * (kernel_size - 1) * 4, &hp));
  BCH_TRY(view_ptr(ctx, "gdn_conv", y, (uint64_t)n_tokens * channels * 4, &yp));
  return launch(ctx, {"gdn_conv", channels, kernel_size, 0},
                [&](hipStream_t s) { run_gdn_conv(s, xp, tp, hp, yp, channels, kernel_size, n_tokens); });
}

extern "C" int bch_gdn_gates(bch_ctx *ctx, bch_view beta, bch_view alpha, bch_view a, bch_view dt_bias,
                             uint32_t n_v_heads, uint32_t n) {
  if (n_v_heads == 0) return fail(BCH_ERR_ARGUMENT, "gdn_gates: no heads");
  float *bp, *ap;
  const float *a_p, *dp;
  BCH_TRY(view_ptr(ctx, "gdn_gates", beta, (uint64_t)n * 4, &bp));
  BCH_TRY(view_ptr(ctx, "gdn_gates", alpha, (uint64_t)n * 4, &ap));
  BCH_TRY(view_ptr(ctx, "gdn_gates", a, (uint64_t)n_v_heads * 4, &a_p));
  BCH_TRY(view_ptr(ctx, "gdn_gates", dt_bias, (uint64_t)n_v_heads * 4, &dp));
  return launch(ctx, {"gdn_gates", n, n_v_heads, 0}, [&](hipStream_t s) { run_gdn_gates(s, bp, ap, a_p, dp, n_v_heads, n); });
}

extern "C" int bch_gdn_recurrence(bch_ctx *ctx, bch_view y, bch_view beta, bch_view decay, bch_view state,
                                  bch_view out, const bch_delta_shape *shape, uint32_t n_tokens, float q_scale) {
  if (!shape) return fail(BCH_ERR_ARGUMENT, "gdn_recurrence: no shape");
  const uint32_t nk = shape->n_k_heads, nv = shape->n_v_heads, dk = shape->k_dim, dv = shape->v_dim;
  if (nk == 0 || nv % nk || (dk != 64 && dk != 128) || dv == 0 || dv % kGdnCols)
    return fail(BCH_ERR_DELTANET_LIMITS,
                "gdn_recurrence: key heads of 64 or 128, value heads a multiple of %d and of the key heads "
                "(got %u/%u heads of %u/%u)", kGdnCols, nk, nv, dk, dv);
  GdnArgs a{};
  const uint64_t conv_dim = 2ull * nk * dk + (uint64_t)nv * dv;
  BCH_TRY(view_ptr(ctx, "gdn_recurrence", y, (uint64_t)n_tokens * conv_dim * 4, &a.y));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence", beta, (uint64_t)n_tokens * nv * 4, &a.beta));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence", decay, (uint64_t)n_tokens * nv * 4, &a.alpha));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence", state, (uint64_t)nv * dk * dv * 4, &a.state));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence", out, (uint64_t)n_tokens * nv * dv * 4, &a.out));
  a.n_k = nk;
  a.n_v = nv;
  a.k_dim = dk;
  a.v_dim = dv;
  a.n_tokens = n_tokens;
  a.q_scale = q_scale;
  a.raw_gates = false;
  if (n_tokens == 0) return BCH_OK;
  return launch(ctx, {"gdn_recurrence", nv, dv, (uint64_t)nv * dk * dv * 8},
                [&](hipStream_t s) { run_gdn_recurrence(s, a); });
}

extern "C" uint64_t bch_gdn_chunk_scratch_floats(const bch_delta_shape *shape, uint32_t n_tokens) {
  if (!shape) return 0;
  return gdn_chunk_scratch_floats(shape->n_v_heads, shape->k_dim, shape->v_dim, n_tokens);
}

extern "C" int bch_gdn_recurrence_chunked(bch_ctx *ctx, bch_view y, bch_view beta, bch_view decay, bch_view state,
                                          bch_view out, const bch_delta_shape *shape, uint32_t n_tokens,
                                          float q_scale, bch_view scratch) {
  if (!shape) return fail(BCH_ERR_ARGUMENT, "gdn_recurrence_chunked: no shape");
  const uint32_t nk = shape->n_k_heads, nv = shape->n_v_heads, dk = shape->k_dim, dv = shape->v_dim;
  if (nk == 0 || nv % nk || (dk != 64 && dk != 128) || dv == 0 || dv % kGdnScanCols || dv > 256)
    return fail(BCH_ERR_DELTANET_LIMITS,
                "gdn_recurrence_chunked: key heads of 64 or 128, value heads of at most 256 and a multiple of %d, "
                "value heads a multiple of the key heads (got %u/%u heads of %u/%u)",
                kGdnScanCols, nk, nv, dk, dv);
  GdnArgs a{};
  const uint64_t conv_dim = 2ull * nk * dk + (uint64_t)nv * dv;
  BCH_TRY(view_ptr(ctx, "gdn_recurrence_chunked", y, (uint64_t)n_tokens * conv_dim * 4, &a.y));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence_chunked", beta, (uint64_t)n_tokens * nv * 4, &a.beta));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence_chunked", decay, (uint64_t)n_tokens * nv * 4, &a.alpha));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence_chunked", state, (uint64_t)nv * dk * dv * 4, &a.state));
  BCH_TRY(view_ptr(ctx, "gdn_recurrence_chunked", out, (uint64_t)n_tokens * nv * dv * 4, &a.out));
  float *sp;
  BCH_TRY(view_ptr(ctx, "gdn_recurrence_chunked", scratch, gdn_chunk_scratch_floats(nv, dk, dv, n_tokens) * 4, &sp));
  if (reinterpret_cast<uintptr_t>(sp) % 16) return fail(BCH_ERR_ARGUMENT, "gdn_recurrence_chunked: scratch not 16-byte aligned");
  a.n_k = nk;
  a.n_v = nv;
  a.k_dim = dk;
  a.v_dim = dv;
  a.n_tokens = n_tokens;
  a.q_scale = q_scale;
  a.raw_gates = false;
  if (n_tokens == 0) return BCH_OK;
  return launch(ctx, {"gdn_recurrence_chunked", nv, dv, (uint64_t)nv * dk * dv * 8},
                [&](hipStream_t s) { run_gdn_chunked(s, a, sp); });
}

extern "C" int bch_gdn_gated_norm(bch_ctx *ctx, bch_view x, bch_view weight, bch_view z, uint32_t v_dim, uint32_t n_rows,
                                  float eps) {
  float *xp;
  const float *wp, *zp;
  BCH_TRY(view_ptr(ctx, "gdn_gated_norm", x, (uint64_t)n_rows * v_dim * 4, &xp));
  BCH_TRY(view_ptr(ctx, "gdn_gated_norm", weight, (uint64_t)v_dim * 4, &wp));
  BCH_TRY(view_ptr(ctx, "gdn_gated_norm", z, (uint64_t)n_rows * v_dim * 4, &zp));
  return launch(ctx, {"gdn_gated_norm", n_rows, v_dim, 0},
                [&](hipStream_t s) { run_gdn_gated_norm(s, xp, wp, zp, v_dim, n_rows, eps); });
}

extern "C" int bch_attention_gate(bch_ctx *ctx, bch_view attn, bch_view q_gate, uint32_t head_dim, uint32_t q_dim,
                                  uint32_t n_tokens) {
  if (head_dim == 0 || q_dim % head_dim) return fail(BCH_ERR_GATE_SHAPE, "attention_gate: %u is not whole heads of %u", q_dim, head_dim);
  float *ap;
  const float *gp;
  BCH_TRY(view_ptr(ctx, "attention_gate", attn, (uint64_t)n_tokens * q_dim * 4, &ap));
  BCH_TRY(view_ptr(ctx, "attention_gate", q_gate, (uint64_t)n_tokens * 2 * q_dim * 4, &gp));
  return launch(ctx, {"attention_gate", n_tokens, q_dim, 0},
                [&](hipStream_t s) { run_attention_gate(s, ap, gp, head_dim, q_dim, n_tokens); });
}
