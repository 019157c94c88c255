// attnres_hip.hip - gfx950 kernels and C ABI of the Fast-AttnRes read.
//
// The read is a bandwidth-bound reduction over S depth sources: every value
// byte is touched once in the forward and once in the backward, so both
// kernels are single streaming passes over HBM with FP32 register state and
// no MFMA (arithmetic intensity is ~3 FP32 flop/byte).
//
// Work decomposition.  A "token group" of G lanes owns one token row; each
// lane owns CH chunks of 8 consecutive BF16 elements (one 16-byte load), the
// chunks of a row interleaved across the group so that one load instruction
// of a wavefront reads a contiguous 16*min(G,64)-byte span:
//     element d of chunk c, lane l:  d = (c*G + l)*8 + e,  e in [0, 8).
// G is 16/32/64 (several tokens per wavefront, reductions by lane shuffles)
// or 128/256 (one token per 2/4 wavefronts, reductions finished in LDS).
// Per-source reductions (key sum of squares, query dot, <v, dO>) therefore
// never leave the compute unit, and the online softmax state (max, sum,
// FP32 accumulator) lives in registers for the whole sweep over sources.
//
// Backward.  For each token: delta = <dO, o> from the saved BF16 output and
// its one-byte refinement (FP32 o to ulp/512, see refine_encode); then per source p = exp(z - max) / sum (from the saved statistics),
// dz = p (<v, dO> - delta), and the value gradient
//     dv = p dO + [key coords] (a q + b v),  a = scale dz / r,  b = -dz z / (R r^2)
// folded in FP32 and stored once as BF16.  dq = sum scale dz k is accumulated
// in registers across the tokens a group visits, reduced over the groups of a
// block in LDS in a fixed order, and the per-block partial rows are summed by
// a second kernel in a fixed order: dq is bit-reproducible.
//
// Reference behaviour followed: src/attnres/_kernels/fixed_tail.py:244-483
// (forward), :485-873 (backward), :875-899 (dq reduction); the list layout of
// src/attnres/_kernels/fla_full_sources.py:164-214, 297-629.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "attnres_hip.h"

namespace {

constexpr int kMaxSources = ATTNRES_MAX_SOURCES;
constexpr int kMaxWidth = ATTNRES_MAX_WIDTH;
constexpr int kBlock = 256;     // threads per workgroup (4 wavefronts)
constexpr int kChunks = 4;      // 16-byte chunks per lane per row
constexpr int kVec = 8;         // BF16 elements per chunk
constexpr int kMaxBwdBlocks = 1024;  // persistent backward grid cap

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- addressing

// Packed [S, N, D] values: row (s, n) at base + s*source_stride + n*row_stride.
struct PackedRows {
  const uint16_t* base;
  int64_t source_stride;
  int64_t row_stride;
  __device__ __forceinline__ const uint16_t* row(int s, int64_t n) const {
    return base + s * source_stride + n * row_stride;
  }
};

// Ordered source list: one base pointer and row stride per list position.
struct ListRows {
  const uint16_t* ptr[kMaxSources];
  int64_t row_stride[kMaxSources];
  __device__ __forceinline__ const uint16_t* row(int s, int64_t n) const {
    return ptr[s] + n * row_stride[s];
  }
};

// Gradients of a packed input: one contiguous [S, N, D] buffer.
struct PackedGrads {
  uint16_t* base;
  int64_t source_stride;  // N * D
  __device__ __forceinline__ uint16_t* row(int s, int64_t n, int d) const {
    return base + s * source_stride + n * d;
  }
};

// Gradients of a source list: one contiguous [N, D] buffer per position.
struct ListGrads {
  uint16_t* ptr[kMaxSources];
  __device__ __forceinline__ uint16_t* row(int s, int64_t n, int d) const {
    return ptr[s] + n * d;
  }
};

template <class Rows>
struct FwdArgs {
  Rows src;
  const uint16_t* query;  // [R] BF16, contiguous
  uint16_t* out;          // [N, D] BF16, contiguous
  int8_t* out_refine;     // [N, D] low-order correction of out (see refine_encode)
  float* logit;           // [N, S]
  float* inv_rms;         // [N, S]
  float* stats;           // [2, N]
  int64_t n_tokens;
  int n_sources;
  int width;
  int rank;
  int vec;                // 1: every row start is 16-byte aligned and D % 8 == 0
  float eps;
  float scale;
};

template <class Rows, class Grads>
struct BwdArgs {
  Rows src;
  Grads grad;
  const uint16_t* query;
  const uint16_t* out;       // [N, D] BF16 forward output, contiguous
  const int8_t* out_refine;  // [N, D] its low-order correction
  const uint16_t* grad_out;  // [N, D] BF16, contiguous
  const float* logit;
  const float* inv_rms;
  const float* stats;
  float* partial;            // [gridDim.x, R] FP32 dq partial rows
  int64_t n_tokens;
  int n_sources;
  int width;
  int rank;
  int vec;
  float scale;
};

// ------------------------------------------------------------- BF16 helpers

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two FP32 values to packed BF16, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, b);
}

__device__ __forceinline__ void unpack_chunk(const u32x4& w, float (&x)[kVec]) {
  x[0] = bf16_lo(w.x); x[1] = bf16_hi(w.x);
  x[2] = bf16_lo(w.y); x[3] = bf16_hi(w.y);
  x[4] = bf16_lo(w.z); x[5] = bf16_hi(w.z);
  x[6] = bf16_lo(w.w); x[7] = bf16_hi(w.w);
}

template <int G>
__device__ __forceinline__ int chunk_start(int c, int lane) { return (c * G + lane) * kVec; }

// Load one row (this lane's chunks) as raw packed BF16 words; elements at or
// beyond D read as +0.  The 16-byte path requires vec (aligned rows, D%8==0).
template <int G>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ row, int lane,
                                         int D, int vec, u32x4 (&raw)[kChunks]) {
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    if (vec) {
      raw[c] = d0 < D ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + d0))
                      : u32x4{0u, 0u, 0u, 0u};
    } else {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = d0 + 2 * j;
        const uint32_t lo = d < D ? static_cast<uint32_t>(row[d]) : 0u;
        const uint32_t hi = d + 1 < D ? static_cast<uint32_t>(row[d + 1]) : 0u;
        w[j] = lo | (hi << 16);
      }
      raw[c] = u32x4{w[0], w[1], w[2], w[3]};
    }
  }
}

template <int G>
__device__ __forceinline__ void load_row_f32(const uint16_t* __restrict__ row, int lane,
                                             int D, int vec, float (&x)[kChunks][kVec]) {
  u32x4 raw[kChunks];
  load_row<G>(row, lane, D, vec, raw);
#pragma unroll
  for (int c = 0; c < kChunks; ++c) unpack_chunk(raw[c], x[c]);
}

template <int G>
__device__ __forceinline__ void store_row(uint16_t* __restrict__ row, int lane, int D, int vec,
                                          const float (&x)[kChunks][kVec]) {
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    if (d0 >= D) continue;
    const u32x4 w = {pack_bf16x2(x[c][0], x[c][1]), pack_bf16x2(x[c][2], x[c][3]),
                     pack_bf16x2(x[c][4], x[c][5]), pack_bf16x2(x[c][6], x[c][7])};
    if (vec) {
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(row + d0));
    } else {
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        if (d0 + e < D) {
          row[d0 + e] = static_cast<uint16_t>((e & 1) ? (ws[e >> 1] >> 16) : (ws[e >> 1] & 0xffffu));
        }
      }
    }
  }
}

// Output refinement.  The backward needs delta = <dO, o> with the FP32 mix o;
// the BF16 output alone leaves a per-token error in delta that accumulates
// in dq over tokens.  The forward therefore also stores one signed byte per
// element: o - bf16(o) in units of ulp(bf16(o))/256 (|o - bf16(o)| <= ulp/2
// under round-to-nearest-even).  Decoding bf16 + q*unit is exact in FP32 and
// recovers o to ulp/512 -- 256x tighter than the BF16 output, at one byte
// per element instead of an FP32 copy's four.  Exponent fields below 16
// (|o| < 2^-111), infinities and NaNs carry no correction.
__device__ __forceinline__ int refine_encode(float o, uint32_t bf16_bits) {
  const int e = static_cast<int>((bf16_bits >> 7) & 0xffu);
  if (e < 16 || e > 254) return 0;
  const float rounded = __uint_as_float(bf16_bits << 16);
  const float inv_unit = __uint_as_float(static_cast<uint32_t>(269 - e) << 23);  // 2^(142-e)
  const float t = rintf((o - rounded) * inv_unit);
  return static_cast<int>(fminf(fmaxf(t, -127.0f), 127.0f));
}

__device__ __forceinline__ float refine_decode(uint32_t bf16_bits, int q) {
  const float rounded = __uint_as_float(bf16_bits << 16);
  const int e = static_cast<int>((bf16_bits >> 7) & 0xffu);
  if (e < 16 || e > 254) return rounded;
  const float unit = __uint_as_float(static_cast<uint32_t>(e - 15) << 23);
  return fmaf(static_cast<float>(q), unit, rounded);
}

// Store this lane's chunks of a BF16 row and of its refinement bytes.
template <int G>
__device__ __forceinline__ void store_row_refined(uint16_t* __restrict__ row, int8_t* __restrict__ refine,
                                                  int lane, int D, int vec,
                                                  const float (&x)[kChunks][kVec]) {
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    if (d0 >= D) continue;
    uint32_t w[4];
    uint32_t r[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = pack_bf16x2(x[c][2 * j], x[c][2 * j + 1]);
      const uint32_t q0 = static_cast<uint32_t>(refine_encode(x[c][2 * j], w[j] & 0xffffu)) & 0xffu;
      const uint32_t q1 = static_cast<uint32_t>(refine_encode(x[c][2 * j + 1], w[j] >> 16)) & 0xffu;
      r[j >> 1] |= (q0 | (q1 << 8)) << (16 * (j & 1));
    }
    if (vec) {
      __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4*>(row + d0));
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      __builtin_nontemporal_store(u32x2{r[0], r[1]}, reinterpret_cast<u32x2*>(refine + d0));
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        if (d0 + e < D) {
          row[d0 + e] = static_cast<uint16_t>((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
          refine[d0 + e] = static_cast<int8_t>((r[e >> 2] >> (8 * (e & 3))) & 0xffu);
        }
      }
    }
  }
}

// Load the FP32 output row reconstructed from BF16 + refinement bytes.
template <int G>
__device__ __forceinline__ void load_row_refined(const uint16_t* __restrict__ row,
                                                 const int8_t* __restrict__ refine, int lane, int D,
                                                 int vec, float (&x)[kChunks][kVec]) {
  u32x4 raw[kChunks];
  load_row<G>(row, lane, D, vec, raw);
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    int8_t q[kVec];
    if (vec) {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 r = d0 < D ? *reinterpret_cast<const u32x2*>(refine + d0) : u32x2{0u, 0u};
#pragma unroll
      for (int e = 0; e < kVec; ++e) q[e] = static_cast<int8_t>(((e < 4 ? r.x : r.y) >> (8 * (e & 3))) & 0xffu);
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) q[e] = d0 + e < D ? refine[d0 + e] : static_cast<int8_t>(0);
    }
    const uint32_t w[4] = {raw[c].x, raw[c].y, raw[c].z, raw[c].w};
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      const uint32_t bits = (e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu);
      x[c][e] = refine_decode(bits, q[e]);
    }
  }
}

// Query scattered onto this lane's row positions: q[d - (D-R)] on the key
// coordinates, +0 elsewhere, so <v, qrow> is the key dot with no masking.
template <int G>
__device__ __forceinline__ void load_query_row(const uint16_t* __restrict__ query, int lane,
                                               int D, int tail0, float (&q)[kChunks][kVec]) {
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      const int d = chunk_start<G>(c, lane) + e;
      q[c][e] = (d >= tail0 && d < D) ? __uint_as_float(static_cast<uint32_t>(query[d - tail0]) << 16)
                                       : 0.0f;
    }
  }
}

// --------------------------------------------------------------- reductions

// Sum NV values over the G lanes of a token group; every lane of the group
// receives the same bits (xor butterflies pair commutative adds, and the
// cross-wavefront stage reads LDS slots in a fixed order).  For G > 64 the
// whole workgroup must call this the same number of times (it contains a
// barrier); `xred` holds two alternating slot sets so one barrier per call
// suffices.
template <int G, int NV>
__device__ __forceinline__ void group_sum(float (&x)[NV], float* xred, int group, int& phase) {
  constexpr int kW = G < 64 ? G : 64;
#pragma unroll
  for (int off = kW / 2; off > 0; off >>= 1) {
#pragma unroll
    for (int i = 0; i < NV; ++i) x[i] += __shfl_xor(x[i], off, kW);
  }
  if constexpr (G > 64) {
    constexpr int kWaves = G / 64;
    constexpr int kGroups = kBlock / G;
    const int wave = (threadIdx.x % G) / 64;
    float* slot = xred + ((phase * kGroups + group) * kWaves) * NV;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
      for (int i = 0; i < NV; ++i) slot[wave * NV + i] = x[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float t = slot[i];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) t += slot[w * NV + i];
      x[i] = t;
    }
    phase ^= 1;
  }
}

template <int G>
constexpr int xred_floats(int nv) {
  return G > 64 ? 2 * (kBlock / G) * (G / 64) * nv : 1;
}

// Does element d belong to the key (the last R coordinates)?
__device__ __forceinline__ bool is_key(int d, int tail0) { return d >= tail0; }

// ------------------------------------------------------------------ forward

template <int G, bool FULLKEY, class Rows>
__global__ void __launch_bounds__(kBlock) attnres_fwd_kernel(const FwdArgs<Rows> a) {
  constexpr int kGroups = kBlock / G;
  __shared__ float xred[xred_floats<G>(2)];
  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int64_t token_id = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const bool valid = token_id < a.n_tokens;
  if constexpr (G <= 64) {
    if (!valid) return;  // no barrier below for in-wavefront groups
  }
  const int64_t token = valid ? token_id : a.n_tokens - 1;
  const int D = a.width;
  const int R = a.rank;
  const int tail0 = D - R;
  const int S = a.n_sources;
  const float inv_R = 1.0f / static_cast<float>(R);
  int phase = 0;

  float q[kChunks][kVec];
  load_query_row<G>(a.query, lane, D, tail0, q);

  float acc[kChunks][kVec];
  float run_max = 0.0f;
  float run_sum = 0.0f;

  u32x4 cur[kChunks];
  load_row<G>(a.src.row(0, token), lane, D, a.vec, cur);
  for (int s = 0; s < S; ++s) {
    u32x4 nxt[kChunks];
    if (s + 1 < S) load_row<G>(a.src.row(s + 1, token), lane, D, a.vec, nxt);

    float v[kChunks][kVec];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) unpack_chunk(cur[c], v[c]);

    float red[2] = {0.0f, 0.0f};  // key sum of squares, <v, q>
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        if (FULLKEY || is_key(chunk_start<G>(c, lane) + e, tail0)) {
          red[0] = fmaf(v[c][e], v[c][e], red[0]);
        }
        red[1] = fmaf(v[c][e], q[c][e], red[1]);
      }
    }
    group_sum<G, 2>(red, xred, group, phase);

    const float inv_rms = 1.0f / sqrtf(red[0] * inv_R + a.eps);
    const float z = red[1] * inv_rms * a.scale;
    if (s == 0) {
      run_max = z;
      run_sum = 1.0f;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[c][e] = v[c][e];
    } else if (z <= run_max) {
      const float w = expf(z - run_max);
      run_sum += w;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[c][e] = fmaf(w, v[c][e], acc[c][e]);
    } else {
      const float w = expf(run_max - z);
      run_sum = fmaf(run_sum, w, 1.0f);
      run_max = z;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[c][e] = fmaf(acc[c][e], w, v[c][e]);
    }
    if (valid && lane == 0) {
      a.logit[token * S + s] = z;
      a.inv_rms[token * S + s] = inv_rms;
    }
#pragma unroll
    for (int c = 0; c < kChunks; ++c) cur[c] = nxt[c];
  }

  const float inv_sum = 1.0f / run_sum;
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[c][e] *= inv_sum;
  if (valid) {
    store_row_refined<G>(a.out + token * D, a.out_refine + token * D, lane, D, a.vec, acc);
    if (lane == 0) {
      a.stats[token] = run_max;
      a.stats[a.n_tokens + token] = inv_sum;
    }
  }
}

// ----------------------------------------------------------------- backward

template <int G>
__device__ __forceinline__ float row_dot(const float (&x)[kChunks][kVec],
                                         const float (&y)[kChunks][kVec]) {
  float t = 0.0f;
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) t = fmaf(x[c][e], y[c][e], t);
  return t;
}

template <int G, bool FULLKEY, class Rows, class Grads>
__global__ void __launch_bounds__(kBlock) attnres_bwd_kernel(const BwdArgs<Rows, Grads> a) {
  constexpr int kGroups = kBlock / G;
  __shared__ float xred[xred_floats<G>(1)];
  __shared__ float dq_lds[kGroups * G * kVec];
  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int D = a.width;
  const int R = a.rank;
  const int tail0 = D - R;
  const int S = a.n_sources;
  const float inv_R = 1.0f / static_cast<float>(R);
  const float scale = a.scale;
  int phase = 0;

  float q[kChunks][kVec];
  load_query_row<G>(a.query, lane, D, tail0, q);
  float dq[kChunks][kVec];
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) dq[c][e] = 0.0f;

  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGroups;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kGroups; base < a.n_tokens; base += stride) {
    const int64_t token_id = base + group;
    const bool valid = token_id < a.n_tokens;
    if constexpr (G <= 64) {
      if (!valid) continue;
    }
    const int64_t token = valid ? token_id : a.n_tokens - 1;

    float g[kChunks][kVec];
    load_row_f32<G>(a.grad_out + token * D, lane, D, a.vec, g);
    float delta[1];
    {
      float o[kChunks][kVec];
      load_row_refined<G>(a.out + token * D, a.out_refine + token * D, lane, D, a.vec, o);
      delta[0] = row_dot<G>(g, o);
    }
    group_sum<G, 1>(delta, xred, group, phase);
    const float run_max = a.stats[token];
    const float inv_sum = a.stats[a.n_tokens + token];

    u32x4 cur[kChunks];
    load_row<G>(a.src.row(0, token), lane, D, a.vec, cur);
    for (int s = 0; s < S; ++s) {
      u32x4 nxt[kChunks];
      if (s + 1 < S) load_row<G>(a.src.row(s + 1, token), lane, D, a.vec, nxt);
      const float z = a.logit[token * S + s];
      const float inv_rms = a.inv_rms[token * S + s];

      float v[kChunks][kVec];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) unpack_chunk(cur[c], v[c]);
      float dw[1] = {row_dot<G>(v, g)};
      group_sum<G, 1>(dw, xred, group, phase);

      const float p = expf(z - run_max) * inv_sum;
      const float dz = p * (dw[0] - delta[0]);
      const float ca = inv_rms * (dz * scale);               // on q, and dq += ca v
      const float cb = -(inv_rms * inv_rms) * (dz * z * inv_R);  // on v (key coords)

      float dv[kChunks][kVec];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) {
          const float direct = p * g[c][e];
          if (FULLKEY || is_key(chunk_start<G>(c, lane) + e, tail0)) {
            dv[c][e] = fmaf(cb, v[c][e], fmaf(ca, q[c][e], direct));
            if (valid) dq[c][e] = fmaf(ca, v[c][e], dq[c][e]);
          } else {
            dv[c][e] = direct;
          }
        }
      }
      if (valid) store_row<G>(a.grad.row(s, token, D), lane, D, a.vec, dv);
#pragma unroll
      for (int c = 0; c < kChunks; ++c) cur[c] = nxt[c];
    }
  }

  // Fixed-order reduction of the groups' dq into this block's partial row.
  float* partial = a.partial + static_cast<int64_t>(blockIdx.x) * R;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
#pragma unroll
    for (int e = 0; e < kVec; ++e) dq_lds[group * (G * kVec) + lane * kVec + e] = dq[c][e];
    __syncthreads();
    for (int j = threadIdx.x; j < G * kVec; j += kBlock) {
      float t = dq_lds[j];
#pragma unroll
      for (int k = 1; k < kGroups; ++k) t += dq_lds[k * (G * kVec) + j];
      const int d = c * G * kVec + j;
      if (d >= tail0 && d < D) partial[d - tail0] = t;
    }
    __syncthreads();
  }
}

// dq[r] = sum over partial rows in a fixed order; FP32 total and BF16 copy.
__global__ void __launch_bounds__(kBlock) attnres_dq_finalize_kernel(
    const float* __restrict__ partial, int64_t rows, int R, float* __restrict__ dq32,
    uint16_t* __restrict__ dq16) {
  __shared__ float lds[kBlock / 64][64];
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  const int slice = threadIdx.x / 64;
  float t = 0.0f;
  if (col < R) {
    for (int64_t r = slice; r < rows; r += kBlock / 64) t += partial[r * R + col];
  }
  lds[slice][threadIdx.x & 63] = t;
  __syncthreads();
  if (slice == 0 && col < R) {
    float total = lds[0][threadIdx.x];
#pragma unroll
    for (int k = 1; k < kBlock / 64; ++k) total += lds[k][threadIdx.x];
    dq32[col] = total;
    dq16[col] = static_cast<uint16_t>(pack_bf16x2(total, 0.0f) & 0xffffu);
  }
}

// ---------------------------------------------------------------- host side

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_shape(int64_t S, int64_t N, int64_t D, int64_t R) {
  if (S < 1 || S > kMaxSources) return fail(ATTNRES_ERR_SHAPE, "n_sources=%lld outside 1..%d", (long long)S, kMaxSources);
  if (N < 1) return fail(ATTNRES_ERR_SHAPE, "n_tokens=%lld must be positive", (long long)N);
  if (D < 1 || D > kMaxWidth) return fail(ATTNRES_ERR_SHAPE, "width=%lld outside 1..%d", (long long)D, kMaxWidth);
  if (R < 1 || R > D) return fail(ATTNRES_ERR_SHAPE, "rank=%lld outside 1..width=%lld", (long long)R, (long long)D);
  return ATTNRES_OK;
}

// Lanes per token: the smallest group whose 32 elements/lane cover the row.
int group_lanes(int64_t D) {
  if (D <= 16 * kChunks * kVec) return 16;
  if (D <= 32 * kChunks * kVec) return 32;
  if (D <= 64 * kChunks * kVec) return 64;
  if (D <= 128 * kChunks * kVec) return 128;
  return 256;
}

int64_t bwd_blocks(int64_t N, int64_t D) {
  const int64_t groups = kBlock / group_lanes(D);
  const int64_t need = (N + groups - 1) / groups;
  return need < kMaxBwdBlocks ? need : kMaxBwdBlocks;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ATTNRES_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return ATTNRES_OK;
}

template <class Rows>
int launch_forward(const FwdArgs<Rows>& a, hipStream_t stream) {
  const int G = group_lanes(a.width);
  const bool full = a.rank == a.width;
  const int groups = kBlock / G;
  const dim3 grid(static_cast<unsigned>((a.n_tokens + groups - 1) / groups));
  const dim3 block(kBlock);
#define ATTNRES_FWD(GG)                                                                   \
  case GG:                                                                                \
    if (full) hipLaunchKernelGGL((attnres_fwd_kernel<GG, true, Rows>), grid, block, 0, stream, a); \
    else hipLaunchKernelGGL((attnres_fwd_kernel<GG, false, Rows>), grid, block, 0, stream, a);     \
    break;
  switch (G) {
    ATTNRES_FWD(16)
    ATTNRES_FWD(32)
    ATTNRES_FWD(64)
    ATTNRES_FWD(128)
    ATTNRES_FWD(256)
  }
#undef ATTNRES_FWD
  return launch_status("attnres forward");
}

template <class Rows, class Grads>
int launch_backward(const BwdArgs<Rows, Grads>& a, float* dq32, uint16_t* dq16,
                    hipStream_t stream) {
  const int G = group_lanes(a.width);
  const bool full = a.rank == a.width;
  const dim3 grid(static_cast<unsigned>(bwd_blocks(a.n_tokens, a.width)));
  const dim3 block(kBlock);
#define ATTNRES_BWD(GG)                                                                             \
  case GG:                                                                                          \
    if (full) hipLaunchKernelGGL((attnres_bwd_kernel<GG, true, Rows, Grads>), grid, block, 0, stream, a); \
    else hipLaunchKernelGGL((attnres_bwd_kernel<GG, false, Rows, Grads>), grid, block, 0, stream, a);     \
    break;
  switch (G) {
    ATTNRES_BWD(16)
    ATTNRES_BWD(32)
    ATTNRES_BWD(64)
    ATTNRES_BWD(128)
    ATTNRES_BWD(256)
  }
#undef ATTNRES_BWD
  int st = launch_status("attnres backward");
  if (st != ATTNRES_OK) return st;
  const dim3 rgrid(static_cast<unsigned>((a.rank + 63) / 64));
  hipLaunchKernelGGL(attnres_dq_finalize_kernel, rgrid, block, 0, stream, a.partial,
                     static_cast<int64_t>(grid.x), a.rank, dq32, dq16);
  return launch_status("attnres dq reduction");
}

int check_scalars(float eps, float scale, bool need_eps) {
  if (need_eps && !(std::isfinite(eps) && eps > 0.0f)) return fail(ATTNRES_ERR_SCALAR, "eps must be finite and positive");
  if (!std::isfinite(scale)) return fail(ATTNRES_ERR_SCALAR, "scale must be finite");
  return ATTNRES_OK;
}

}  // namespace

// ------------------------------------------------------------------- C ABI

extern "C" {

const char* attnres_hip_version(void) { return "1.0.0"; }

const char* attnres_hip_last_error(void) { return g_error; }

int64_t attnres_hip_dq_workspace_elems(int64_t n_tokens, int64_t width, int64_t rank) {
  if (check_shape(1, n_tokens, width, rank) != ATTNRES_OK) return -1;
  return (bwd_blocks(n_tokens, width) + 1) * rank;
}

int attnres_hip_packed_forward(const void* values, int64_t source_stride, int64_t row_stride,
                               int64_t n_sources, int64_t n_tokens, int64_t width,
                               const void* query, int64_t rank, float eps, float scale,
                               void* out, int8_t* out_refine, float* logit, float* inv_rms,
                               float* stats, void* stream) {
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  if (!values || !query || !out || !out_refine || !logit || !inv_rms || !stats)
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to attnres_hip_packed_forward");
  if (source_stride < 0 || row_stride < 0) return fail(ATTNRES_ERR_STRIDE, "negative stride");
  if ((st = check_scalars(eps, scale, true))) return st;
  FwdArgs<PackedRows> a{};
  a.src = PackedRows{static_cast<const uint16_t*>(values), source_stride, row_stride};
  a.query = static_cast<const uint16_t*>(query);
  a.out = static_cast<uint16_t*>(out);
  a.out_refine = out_refine;
  a.logit = logit;
  a.inv_rms = inv_rms;
  a.stats = stats;
  a.n_tokens = n_tokens;
  a.n_sources = static_cast<int>(n_sources);
  a.width = static_cast<int>(width);
  a.rank = static_cast<int>(rank);
  a.vec = width % kVec == 0 && aligned16(values) && aligned16(out) &&
          (source_stride % kVec == 0 || n_sources == 1) && (row_stride % kVec == 0 || n_tokens == 1);
  a.eps = eps;
  a.scale = scale;
  return launch_forward(a, static_cast<hipStream_t>(stream));
}

int attnres_hip_packed_backward(const void* values, int64_t source_stride, int64_t row_stride,
                                int64_t n_sources, int64_t n_tokens, int64_t width,
                                const void* query, int64_t rank, float scale, const void* out,
                                const int8_t* out_refine, const void* grad_out,
                                const float* logit, const float* inv_rms, const float* stats,
                                void* grad_values, void* grad_query, float* dq_workspace,
                                int64_t dq_workspace_elems, void* stream) {
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  if (!values || !query || !out || !out_refine || !grad_out || !logit || !inv_rms || !stats ||
      !grad_values || !grad_query || !dq_workspace)
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to attnres_hip_packed_backward");
  if (source_stride < 0 || row_stride < 0) return fail(ATTNRES_ERR_STRIDE, "negative stride");
  if ((st = check_scalars(1.0f, scale, false))) return st;
  const int64_t need = attnres_hip_dq_workspace_elems(n_tokens, width, rank);
  if (dq_workspace_elems < need)
    return fail(ATTNRES_ERR_WORKSPACE, "dq workspace has %lld elements, needs %lld",
                (long long)dq_workspace_elems, (long long)need);
  BwdArgs<PackedRows, PackedGrads> a{};
  a.src = PackedRows{static_cast<const uint16_t*>(values), source_stride, row_stride};
  a.grad = PackedGrads{static_cast<uint16_t*>(grad_values), n_tokens * width};
  a.query = static_cast<const uint16_t*>(query);
  a.out = static_cast<const uint16_t*>(out);
  a.out_refine = out_refine;
  a.grad_out = static_cast<const uint16_t*>(grad_out);
  a.logit = logit;
  a.inv_rms = inv_rms;
  a.stats = stats;
  a.partial = dq_workspace;
  a.n_tokens = n_tokens;
  a.n_sources = static_cast<int>(n_sources);
  a.width = static_cast<int>(width);
  a.rank = static_cast<int>(rank);
  a.vec = width % kVec == 0 && aligned16(values) && aligned16(out) && aligned16(grad_out) &&
          aligned16(grad_values) && (source_stride % kVec == 0 || n_sources == 1) &&
          (row_stride % kVec == 0 || n_tokens == 1);
  a.scale = scale;
  float* dq32 = dq_workspace + (need - rank);
  return launch_backward(a, dq32, static_cast<uint16_t*>(grad_query), static_cast<hipStream_t>(stream));
}

int attnres_hip_sources_forward(const void* const* sources, const int64_t* row_strides,
                                int64_t n_sources, int64_t n_tokens, int64_t width,
                                const void* query, int64_t rank, float eps, float scale, void* out,
                                int8_t* out_refine, float* logit, float* inv_rms, float* stats,
                                void* stream) {
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  if (!sources || !row_strides || !query || !out || !out_refine || !logit || !inv_rms || !stats)
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to attnres_hip_sources_forward");
  if ((st = check_scalars(eps, scale, true))) return st;
  FwdArgs<ListRows> a{};
  bool vec = width % kVec == 0 && aligned16(out);
  for (int64_t s = 0; s < n_sources; ++s) {
    if (!sources[s]) return fail(ATTNRES_ERR_NULL_POINTER, "source %lld is null", (long long)s);
    if (row_strides[s] < 0) return fail(ATTNRES_ERR_STRIDE, "source %lld has a negative row stride", (long long)s);
    a.src.ptr[s] = static_cast<const uint16_t*>(sources[s]);
    a.src.row_stride[s] = row_strides[s];
    vec = vec && aligned16(sources[s]) && (row_strides[s] % kVec == 0 || n_tokens == 1);
  }
  a.query = static_cast<const uint16_t*>(query);
  a.out = static_cast<uint16_t*>(out);
  a.out_refine = out_refine;
  a.logit = logit;
  a.inv_rms = inv_rms;
  a.stats = stats;
  a.n_tokens = n_tokens;
  a.n_sources = static_cast<int>(n_sources);
  a.width = static_cast<int>(width);
  a.rank = static_cast<int>(rank);
  a.vec = vec;
  a.eps = eps;
  a.scale = scale;
  return launch_forward(a, static_cast<hipStream_t>(stream));
}

int attnres_hip_sources_backward(const void* const* sources, const int64_t* row_strides,
                                 int64_t n_sources, int64_t n_tokens, int64_t width,
                                 const void* query, int64_t rank, float scale, const void* out,
                                 const int8_t* out_refine, const void* grad_out,
                                 const float* logit, const float* inv_rms, const float* stats,
                                 void* const* grad_sources, void* grad_query, float* dq_workspace,
                                 int64_t dq_workspace_elems, void* stream) {
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  if (!sources || !row_strides || !query || !out || !out_refine || !grad_out || !logit ||
      !inv_rms || !stats || !grad_sources || !grad_query || !dq_workspace)
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to attnres_hip_sources_backward");
  if ((st = check_scalars(1.0f, scale, false))) return st;
  const int64_t need = attnres_hip_dq_workspace_elems(n_tokens, width, rank);
  if (dq_workspace_elems < need)
    return fail(ATTNRES_ERR_WORKSPACE, "dq workspace has %lld elements, needs %lld",
                (long long)dq_workspace_elems, (long long)need);
  BwdArgs<ListRows, ListGrads> a{};
  bool vec = width % kVec == 0 && aligned16(out) && aligned16(grad_out);
  for (int64_t s = 0; s < n_sources; ++s) {
    if (!sources[s] || !grad_sources[s])
      return fail(ATTNRES_ERR_NULL_POINTER, "source %lld or its gradient is null", (long long)s);
    if (row_strides[s] < 0) return fail(ATTNRES_ERR_STRIDE, "source %lld has a negative row stride", (long long)s);
    a.src.ptr[s] = static_cast<const uint16_t*>(sources[s]);
    a.src.row_stride[s] = row_strides[s];
    a.grad.ptr[s] = static_cast<uint16_t*>(grad_sources[s]);
    vec = vec && aligned16(sources[s]) && aligned16(grad_sources[s]) &&
          (row_strides[s] % kVec == 0 || n_tokens == 1);
  }
  a.query = static_cast<const uint16_t*>(query);
  a.out = static_cast<const uint16_t*>(out);
  a.out_refine = out_refine;
  a.grad_out = static_cast<const uint16_t*>(grad_out);
  a.logit = logit;
  a.inv_rms = inv_rms;
  a.stats = stats;
  a.partial = dq_workspace;
  a.n_tokens = n_tokens;
  a.n_sources = static_cast<int>(n_sources);
  a.width = static_cast<int>(width);
  a.rank = static_cast<int>(rank);
  a.vec = vec;
  a.scale = scale;
  float* dq32 = dq_workspace + (need - rank);
  return launch_backward(a, dq32, static_cast<uint16_t*>(grad_query), static_cast<hipStream_t>(stream));
}

}  // extern "C"
