// attnres_kernels.hip - gfx950 kernels of the Fast-AttnRes read.
//
// Compiled once per row geometry (ATTNRES_LANES, ATTNRES_CHUNKS); the C ABI
// in attnres_hip.hip dispatches to the instantiations declared in
// attnres_internal.h.
//
// The read is a bandwidth-bound reduction over S depth sources: every value
// byte is touched once in the forward and once in the backward, so both
// kernels are single streaming passes over HBM with FP32 register state and
// no MFMA (arithmetic intensity is ~3 FP32 flop/byte).
//
// Work decomposition.  A "token group" of G lanes owns one token row; each
// lane owns CH chunks of 8 consecutive BF16 elements (one 16-byte load), the
// chunks of a row interleaved across the group so that one load instruction
// of a wavefront reads a contiguous span:
//     element d of chunk c, lane l:  d = (c*G + l)*8 + e,  e in [0, 8).
// G is 16/32/64 (one or several tokens per wavefront; sums over the group are
// DPP butterflies inside 16-lane rows plus lane reads across rows) or 256
// (one token per workgroup for D > 4096; the four wave sums meet in LDS).
//
// Forward.  Per token, the S source rows stream through a ring of NB rows
// held in registers (NB loads in flight per group).  For each source the
// packed BF16 words feed v_dot2_f32_bf16 for the key sum of squares and the
// query dot; the online softmax (running max, running sum, FP32 accumulator
// of the full row) is updated; the per-source logit and 1/rms and the
// per-token (max, 1/sum) are saved for the backward.
//
// Backward.  A grid of up to two resident grids; group g takes tokens g,
// g + groups, ... so that the groups work on neighbouring tokens at any time
// and walk the sources roughly in step.  The ring of value rows crosses token boundaries;
// at each new token the group loads dO and the saved output (BF16 plus one
// refinement byte per element, see refine_encode) and forms
// delta = <dO, o>.  Per item: dw = <v, dO>, p = exp(z - max) / sum,
// dz = p (dw - delta), and
//     dv = p dO + [key coords] (a q + b v),  a = scale dz / r,  b = -dz z / (R r^2)
// folded in FP32 and stored once as BF16.  dq = sum scale dz k accumulates in
// registers; each workgroup reduces its groups in LDS in a fixed order to
// one partial row, and one small kernel sums the partial rows in a fixed
// order, so dq is bit-reproducible run to run.  The ring holds one value row
// per group, or two for aligned 4-chunk rows where that does not spill (see
// launch_bwd).
//
// Variants of the backward.  For S <= 6 (the save/recompute policy) a group
// holds all S rows of its token and takes delta = sum_s p_s dw_s from them,
// so the forward stores no refinement and the backward reads no saved output
// (attnres_bwd_recompute_kernel).  Reads of up to 16 sources whose key is a
// suffix of whole chunk columns (R = 512 or 1024 of D = 2048 or 4096), and of
// up to 12 with D = R = 2048, do the same while streaming their rows: only the
// key chunks of a token's rows are held until delta is complete
// (attnres_bwd_keyres_kernel).  The accumulating variant adds dv to
// existing gradient rows (BF16, or FP32 sums for a source bank).  The
// coefficient variant writes no dv at all, only the per-token terms p, a, b;
// a source bank later forms each source's gradient once from the dO rows of
// every read that saw it (attnres_gather_kernel).
//
// Reference behaviour followed: src/attnres/_kernels/fixed_tail.py:244-483
// (forward), :485-873 (backward), :875-899 (dq reduction); the list layout of
// src/attnres/_kernels/fla_full_sources.py:164-214, 297-629.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

#include "attnres_internal.h"

namespace attnres_hip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------- BF16 helpers

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two FP32 values to packed BF16, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, b);
}

// acc + a.lo*b.lo + a.hi*b.hi on packed BF16 pairs (v_dot2_f32_bf16): the
// products are exact in FP32 and the sum is rounded as an FP32 addition.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), acc, false);
}

template <int G>
__device__ __forceinline__ int chunk_start(int c, int lane) { return (c * G + lane) * kVec; }

// Load one row (this lane's chunks) as raw packed BF16 words.  Every load is
// unconditional: a chunk that starts at or beyond D reads the row's first
// chunk instead, and callers neutralise such lanes with the word masks of
// key_masks / range_masks (branch-free loads keep several rows in flight;
// a conditional load would join control flow and force a wait for it).
// VEC requires 16-byte aligned rows and D % 8 == 0 (so D >= 8).
template <int G, int CH, bool VEC>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ row, int lane, int D,
                                         u32x4 (&raw)[CH]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    if constexpr (VEC) {
      const int at = d0 < D ? d0 : 0;
      raw[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + at));
    } else {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = d0 + 2 * j;
        const uint32_t lo = row[d < D ? d : D - 1];
        const uint32_t hi = row[d + 1 < D ? d + 1 : D - 1];
        w[j] = lo | (hi << 16);
      }
      raw[c] = u32x4{w[0], w[1], w[2], w[3]};
    }
  }
}

// Stores of rows whose base address is the same across the wavefront
// (token groups of 64 lanes and more) are buffer stores with the sc1 and nt
// cache bits: non-temporal, device scope.  The rows they write (outputs,
// refinement bytes, value gradients) are read only by later kernels.
// Measured on MI355X against the nt-only stores of __builtin_nontemporal_store:
// c4 backward 503 -> 487 us, c3 backward 838 -> 829 us, c2 unchanged.
// Narrower groups (several tokens per wavefront) keep the nt-only stores: a
// buffer resource needs a wave-uniform base.
constexpr int kStoreScNt = 16 | 2;  // cache policy: SC1 | NT

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_resource(const void* row, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(row), static_cast<short>(0), bytes, 0x00020000);
}

template <int G, bool VEC>
__device__ __forceinline__ void store_chunk(uint16_t* __restrict__ row, int d0, int D, const u32x4& w) {
  if constexpr (VEC && G >= 64) {
    __builtin_amdgcn_raw_buffer_store_b128(w, row_resource(row, 2 * D), 2 * d0, 0, kStoreScNt);
  } else if constexpr (VEC) {
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
  const float rounded = __uint_as_float(bf16_bits << 16);
  // 2^(142-e) for 16 <= e <= 254; the clamped exponent keeps the factor a
  // normal float for every e, and the select below drops the other cases.
  const int ec = min(max(e, 16), 254);
  const float inv_unit = __uint_as_float(static_cast<uint32_t>(269 - ec) << 23);
  const float t = fminf(fmaxf(rintf((o - rounded) * inv_unit), -127.0f), 127.0f);
  return (e >= 16 && e <= 254) ? static_cast<int>(t) : 0;
}

// Store this lane's chunks of a BF16 row and (REFINE) of its refinement bytes.
template <int G, int CH, bool NOMASK, bool VEC, bool REFINE>
__device__ __forceinline__ void store_row_refined(uint16_t* __restrict__ row, int8_t* __restrict__ refine,
                                                  int lane, int D, const float (&x)[CH][kVec]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    if (!NOMASK && d0 >= D) continue;
    uint32_t w[4];
    uint32_t r[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = pack_bf16x2(x[c][2 * j], x[c][2 * j + 1]);
      if constexpr (REFINE) {
        const uint32_t q0 = static_cast<uint32_t>(refine_encode(x[c][2 * j], w[j] & 0xffffu)) & 0xffu;
        const uint32_t q1 = static_cast<uint32_t>(refine_encode(x[c][2 * j + 1], w[j] >> 16)) & 0xffu;
        r[j >> 1] |= (q0 | (q1 << 8)) << (16 * (j & 1));
      }
    }
    store_chunk<G, VEC>(row, d0, D, u32x4{w[0], w[1], w[2], w[3]});
    if constexpr (!REFINE) {
    } else if constexpr (VEC && G >= 64) {
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{r[0], r[1]}, row_resource(refine, D), d0, 0, kStoreScNt);
    } else if constexpr (VEC) {
      __builtin_nontemporal_store(u32x2{r[0], r[1]}, reinterpret_cast<u32x2*>(refine + d0));
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        if (d0 + e < D) refine[d0 + e] = static_cast<int8_t>((r[e >> 2] >> (8 * (e & 3))) & 0xffu);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // encode one chunk at a time (register pressure)
  }
}

// Query words on this lane's row positions: packed BF16 q[d - (D-R)] on the
// key coordinates, +0 elsewhere (including d >= D).  The loads are
// unconditional (clamped index) and masked afterwards, so none of them sits
// behind a branch.
template <int G, int CH>
__device__ __forceinline__ void load_query_words(const uint16_t* __restrict__ query, int lane, int D,
                                                 int tail0, uint32_t (&qw)[CH][4]) {
  const int R = D - tail0;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = chunk_start<G>(c, lane) + 2 * j;
      const uint32_t lo = query[min(max(d - tail0, 0), R - 1)];
      const uint32_t hi = query[min(max(d + 1 - tail0, 0), R - 1)];
      const uint32_t mask = ((d >= tail0 && d < D) ? 0x0000ffffu : 0u) |
                            ((d + 1 >= tail0 && d + 1 < D) ? 0xffff0000u : 0u);
      qw[c][j] = (lo | (hi << 16)) & mask;
    }
  }
}

// Word masks selecting the key coordinates (D-R <= d < D) of this lane's words.
template <int G, int CH>
__device__ __forceinline__ void key_masks(int lane, int D, int tail0, uint32_t (&km)[CH][4]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = chunk_start<G>(c, lane) + 2 * j;
      km[c][j] = ((d >= tail0 && d < D) ? 0x0000ffffu : 0u) |
                 ((d + 1 >= tail0 && d + 1 < D) ? 0xffff0000u : 0u);
    }
  }
}

// Zero the words of this lane's chunks that lie at or beyond D.
template <int G, int CH>
__device__ __forceinline__ void mask_range(int lane, int D, u32x4 (&x)[CH]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int d = chunk_start<G>(c, lane);
    x[c].x &= (d < D ? 0x0000ffffu : 0u) | (d + 1 < D ? 0xffff0000u : 0u);
    x[c].y &= (d + 2 < D ? 0x0000ffffu : 0u) | (d + 3 < D ? 0xffff0000u : 0u);
    x[c].z &= (d + 4 < D ? 0x0000ffffu : 0u) | (d + 5 < D ? 0xffff0000u : 0u);
    x[c].w &= (d + 6 < D ? 0x0000ffffu : 0u) | (d + 7 < D ? 0xffff0000u : 0u);
  }
}

// --------------------------------------------------------------- reductions

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Sum over the W lanes of a token group inside one wavefront (W = 16, 32 or
// 64, groups aligned to W).  DPP quad permutations and row mirrors sum each
// 16-lane row; rows are combined from lane reads.  Every lane of the group
// receives the same bits: each step adds a pair of partial sums that all
// receiving lanes see in one of the two orders of a commutative add.
template <int W>
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp<0xb1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4e>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  x += dpp<0x140>(x);  // row_mirror
  if constexpr (W == 16) {
    return x;
  } else if constexpr (W == 32) {
    const float lo = lane_value(x, 0) + lane_value(x, 16);
    const float hi = lane_value(x, 32) + lane_value(x, 48);
    return (threadIdx.x & 32) ? hi : lo;
  } else {
    static_assert(W == 64, "group width");
    return (lane_value(x, 0) + lane_value(x, 16)) + (lane_value(x, 32) + lane_value(x, 48));
  }
}

// Sum NV values over the G lanes of a token group.  For G > 64 the group is
// the whole workgroup: the wave sums meet in LDS (every thread must make the
// same sequence of calls; `xred` holds two alternating slot sets so one
// barrier per call suffices).
template <int G, int NV>
__device__ __forceinline__ void group_sum(float (&x)[NV], float* xred, int& phase) {
#pragma unroll
  for (int i = 0; i < NV; ++i) x[i] = wave_sum<(G < 64 ? G : 64)>(x[i]);
  if constexpr (G > 64) {
    constexpr int kWaves = G / 64;
    const int wave = threadIdx.x / 64;
    float* slot = xred + phase * kWaves * NV;
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
  return G > 64 ? 2 * (G / 64) * nv : 1;
}

// ------------------------------------------------------------------ forward

// Index of this thread's token group.  For G >= 64 a group is one or more
// whole wavefronts, and readfirstlane tells the compiler so: group-level
// cursors, loop bounds and branches then live in scalar registers.
template <int G>
__device__ __forceinline__ int group_index() {
  if constexpr (G >= 64) {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / G);
  } else {
    return static_cast<int>(threadIdx.x) / G;
  }
}

// Cursor over a group's (token, source) items in token-major order.
struct ItemCursor {
  int64_t token;
  int source;
  int64_t stride = 1;  // tokens between a group's consecutive tokens
  __device__ __forceinline__ void advance(int S) {
    if (++source == S) {
      source = 0;
      token += stride;
    }
  }
};

// Refill a ring slot with the row of `at`, or -- past the end of the range --
// with a load every lane points at one live address (a single cache line), so
// that each slot is refilled unconditionally: a conditional refill would make
// the compiler wait for all outstanding loads before every slot is used.
template <int G, int CH, bool VEC, class Rows>
__device__ __forceinline__ void refill(const Rows& src, const ItemCursor& at, bool live, const uint16_t* idle,
                                       int lane, int D, u32x4 (&slot)[CH]) {
  if constexpr (VEC) {
    const uint16_t* row = live ? src.row(at.source, at.token) : idle;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int d0 = chunk_start<G>(c, lane);
      const int offset = (live && d0 < D) ? d0 : 0;
      slot[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + offset));
    }
  } else {
    load_row<G, CH, VEC>(live ? src.row(at.source, at.token) : idle, lane, D, slot);
  }
}

// NOMASK: R == D and D == G*CH*8, so every lane position is an in-range key
// coordinate and no word masks are needed.
//
// Group g takes tokens g, g + groups, ... and streams their rows through the
// ring without draining it between tokens (launched with a persistent grid
// for small S, else with one token per group; see launch_fwd).
template <int G, int CH, int NB, bool NOMASK, bool VEC, class Rows>
__global__ void __launch_bounds__(kBlock) attnres_fwd_kernel(const FwdArgs<Rows> a) {
  static_assert(G <= 64 || G == kBlock, "a wide group is the whole workgroup");
  constexpr int kGroups = kBlock / G;
  __shared__ float xred[xred_floats<G>(2)];
  const int lane = threadIdx.x % G;
  const int group = group_index<G>();
  const int D = a.width;
  const int tail0 = D - a.rank;
  const int S = a.n_sources;
  const float inv_R = 1.0f / static_cast<float>(a.rank);
  int phase = 0;

  // Group gid takes tokens gid, gid + groups, ... (see the backward kernel);
  // items are counted per group: item i is source i % S of the group's
  // token i / S.
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const int64_t groups = static_cast<int64_t>(gridDim.x) * kGroups;
  const int64_t my_tokens = gid < a.n_tokens ? (a.n_tokens - 1 - gid) / groups + 1 : 0;
  if (my_tokens == 0) return;  // whole group idle (no barrier follows for it)

  uint32_t qw[CH][4];
  load_query_words<G, CH>(a.query, lane, D, tail0, qw);
  uint32_t km[CH][4];
  if constexpr (!NOMASK) key_masks<G, CH>(lane, D, tail0, km);

  const int64_t last = my_tokens * S;
  const uint16_t* idle = a.src.row(0, gid);
  ItemCursor ahead{gid, 0, groups};
  int64_t ahead_item = 0;
  u32x4 ring[NB][CH];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const bool live = ahead_item < last;
    refill<G, CH, VEC>(a.src, ahead, live, idle, lane, D, ring[j]);
    if (live) {
      ++ahead_item;
      ahead.advance(S);
    }
  }

  // acc needs no reset between tokens: with run_max = -inf the first
  // source of a token rescales the old (finite) contents by exp(-inf) = 0.
  float acc[CH][kVec];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[c][e] = 0.0f;
  float run_max = -INFINITY;
  float run_sum = 0.0f;
  ItemCursor at{gid, 0, groups};

  // One item: the row in ring slot j.  `refill_slot` is false only in the
  // remainder after the last full round, where every row is already loaded.
  auto step = [&](int j, bool refill_slot) __attribute__((always_inline)) {
    const int s = at.source;
    const int64_t token = at.token;
    float red[2] = {0.0f, 0.0f};  // key sum of squares, <key, q>
    {
      float ss1 = 0.0f, qd1 = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t w[4] = {ring[j][c].x, ring[j][c].y, ring[j][c].z, ring[j][c].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t kw = NOMASK ? w[k] : (w[k] & km[c][k]);
          if (k & 1) {
            ss1 = dot2(kw, kw, ss1);
            qd1 = dot2(kw, qw[c][k], qd1);
          } else {
            red[0] = dot2(kw, kw, red[0]);
            red[1] = dot2(kw, qw[c][k], red[1]);
          }
        }
      }
      red[0] += ss1;
      red[1] += qd1;
    }
    group_sum<G, 2>(red, xred, phase);
    const float inv_rms = rsqrtf(fmaf(red[0], inv_R, a.eps));
    const float z = red[1] * inv_rms * a.scale;

    // Online softmax.  A new maximum first rescales the accumulator in place
    // (a group-uniform branch taken on the sources that raise the maximum);
    // then every source adds exp(z - max) * v with one FMA per element.  A
    // single update path keeps the accumulator in one set of registers.
    if (z > run_max) {
      const float alpha = __expf(run_max - z);  // 0 for the first source of a token
      run_sum *= alpha;
      run_max = z;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[c][e] *= alpha;
    }
    {
      const float w = __expf(z - run_max);
      run_sum += w;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t wd[4] = {ring[j][c].x, ring[j][c].y, ring[j][c].z, ring[j][c].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[c][2 * k] = fmaf(w, bf16_lo(wd[k]), acc[c][2 * k]);
          acc[c][2 * k + 1] = fmaf(w, bf16_hi(wd[k]), acc[c][2 * k + 1]);
        }
      }
    }
    if (lane == 0) {
      a.logit[token * S + s] = z;
      a.inv_rms[token * S + s] = inv_rms;
    }

    if (refill_slot) {
      // The slot is refilled only after its last use: without the barrier the
      // scheduler hoists the load and keeps two copies of the slot live.
      __builtin_amdgcn_sched_barrier(0);
      const bool live = ahead_item < last;
      refill<G, CH, VEC>(a.src, ahead, live, idle, lane, D, ring[j]);
      if (live) {
        ++ahead_item;
        ahead.advance(S);
      }
    }

    if (s == S - 1) {  // token complete: normalise and store the output row
      // Normalised in place: the next token's first source rescales acc by 0.
      const float inv_sum = 1.0f / run_sum;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[c][e] *= inv_sum;
      // No refinement under the recompute policy (out_refine == nullptr, a
      // kernel argument: the branch is uniform over the grid).
      if (a.out_refine) {
        store_row_refined<G, CH, NOMASK, VEC, true>(a.out + token * D, a.out_refine + token * D, lane, D, acc);
      } else {
        store_row_refined<G, CH, NOMASK, VEC, false>(a.out + token * D, nullptr, lane, D, acc);
      }
      if (lane == 0) {
        a.stats[token] = run_max;
        a.stats[a.n_tokens + token] = inv_sum;
      }
      run_max = -INFINITY;
      run_sum = 0.0f;
    }
    at.advance(S);
  };

  // Full rounds refill every slot (with an idle load past the end), so the
  // loop body has no exit test between slots: any such path back to the loop
  // head would make the compiler wait there for all outstanding loads.
  const int64_t items = last;
  const int64_t rounds = items / NB;
  const int rem = static_cast<int>(items - rounds * NB);
  for (int64_t r = 0; r < rounds; ++r) {
#pragma unroll
    for (int j = 0; j < NB; ++j) step(j, true);
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (j < rem) step(j, false);
  }
}

// Token-block forward: a group owns T consecutive tokens and streams their
// rows source-major -- items (s, t) for s = 0..S-1, t = 0..T-1 -- through a
// ring of T * NBT slots; slot j always serves token j % T.  The rows a group
// has in flight are then one source's rows of adjacent tokens (a contiguous
// span) rather than several sources of one token, rows a power-of-two source
// stride apart that can fall into the same DRAM banks.  Per-token arithmetic
// is the one-token kernel's (same sums in the same order): bit-identical
// results.  Used at D = R = 2048 with T = 2, NBT = 2 (four rows in flight,
// two per token, 206 VGPRs, two waves per SIMD) for 5 <= S <= 12, and with
// T = 4, NBT = 1 (one row per token, 259 registers, one wave per SIMD) for
// S >= 24; with T = 2, NBT = 1 for 64 lanes of 8 chunks (2048 < D <= 4096,
// masked or not) from S = 13, for shorter rows of 64 lanes of 4 chunks
// (1024 < D < 2048) and for workgroup-wide groups (4096 < D <= 8192) from
// S = 5; with 32-lane groups (two per wavefront) for 128 < D <= 512 (T = 2,
// NBT = 2) from S = 5 and for 512 < D < 1024 (T = 2, NBT = 1) from S = 9; see
// launch_fwd for the measurements.  T = 4 forced to two waves
// per SIMD (256 VGPRs) took 317-349 against 299-323 us at c2; the query words
// read from LDS instead of registers made no difference.
// Like the token-block backward, its timing is sensitive to code generation:
// changes are measured before they are kept.
template <int G, int CH, int T, int NBT, bool NOMASK, bool VEC, class Rows>
__global__ void __launch_bounds__(kBlock) attnres_fwd_block_kernel(const FwdArgs<Rows> a) {
  static_assert(G <= 64 || G == kBlock, "a wide group is the whole workgroup");
  constexpr int kGroups = kBlock / G;
  constexpr int NB = T * NBT;
  __shared__ float xred[xred_floats<G>(2)];
  const int lane = threadIdx.x % G;
  const int group = group_index<G>();
  const int D = a.width;
  const int tail0 = D - a.rank;
  const int S = a.n_sources;
  const int64_t N = a.n_tokens;
  const float inv_R = 1.0f / static_cast<float>(a.rank);
  int phase = 0;

  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const int64_t tok0 = gid * T;
  if (tok0 >= N) return;  // whole group idle
  int64_t tok[T];
  bool valid[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    valid[t] = tok0 + t < N;
    tok[t] = valid[t] ? tok0 + t : N - 1;
  }

  uint32_t qw[CH][4];
  load_query_words<G, CH>(a.query, lane, D, tail0, qw);
  uint32_t km[CH][4];
  if constexpr (!NOMASK) key_masks<G, CH>(lane, D, tail0, km);

  const uint16_t* idle = a.src.row(0, tok[0]);
  u32x4 ring[NB][CH];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int s = j / T;
    const ItemCursor at{tok[j % T], s < S ? s : 0, 1};
    refill<G, CH, VEC>(a.src, at, s < S, idle, lane, D, ring[j]);
  }

  float acc[T][CH][kVec];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < kVec; ++e) acc[t][c][e] = 0.0f;
  float run_max[T], run_sum[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    run_max[t] = -INFINITY;
    run_sum[t] = 0.0f;
  }

  auto step = [&](int j, int s, bool refill_slot) __attribute__((always_inline)) {
    const int t = j % T;
    const int64_t token = tok[t];
    float red[2] = {0.0f, 0.0f};
    {
      float ss1 = 0.0f, qd1 = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t w[4] = {ring[j][c].x, ring[j][c].y, ring[j][c].z, ring[j][c].w};
        const uint32_t qv[4] = {qw[c][0], qw[c][1], qw[c][2], qw[c][3]};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t kw = NOMASK ? w[k] : (w[k] & km[c][k]);
          if (k & 1) {
            ss1 = dot2(kw, kw, ss1);
            qd1 = dot2(kw, qv[k], qd1);
          } else {
            red[0] = dot2(kw, kw, red[0]);
            red[1] = dot2(kw, qv[k], red[1]);
          }
        }
      }
      red[0] += ss1;
      red[1] += qd1;
    }
    group_sum<G, 2>(red, xred, phase);
    const float inv_rms = rsqrtf(fmaf(red[0], inv_R, a.eps));
    const float z = red[1] * inv_rms * a.scale;
    if (z > run_max[t]) {
      const float alpha = __expf(run_max[t] - z);
      run_sum[t] *= alpha;
      run_max[t] = z;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[t][c][e] *= alpha;
    }
    {
      const float w = __expf(z - run_max[t]);
      run_sum[t] += w;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t wd[4] = {ring[j][c].x, ring[j][c].y, ring[j][c].z, ring[j][c].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[t][c][2 * k] = fmaf(w, bf16_lo(wd[k]), acc[t][c][2 * k]);
          acc[t][c][2 * k + 1] = fmaf(w, bf16_hi(wd[k]), acc[t][c][2 * k + 1]);
        }
      }
    }
    if (lane == 0 && valid[t]) {
      a.logit[token * S + s] = z;
      a.inv_rms[token * S + s] = inv_rms;
    }
    if (refill_slot) {
      __builtin_amdgcn_sched_barrier(0);
      const int sn = s + NBT;
      const ItemCursor at{token, sn < S ? sn : 0, 1};
      refill<G, CH, VEC>(a.src, at, sn < S, idle, lane, D, ring[j]);
    }
    if (s == S - 1) {
      const float inv_sum = 1.0f / run_sum[t];
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[t][c][e] *= inv_sum;
      if (valid[t]) {
        if (a.out_refine) {
          store_row_refined<G, CH, NOMASK, VEC, true>(a.out + token * D, a.out_refine + token * D, lane, D, acc[t]);
        } else {
          store_row_refined<G, CH, NOMASK, VEC, false>(a.out + token * D, nullptr, lane, D, acc[t]);
        }
        if (lane == 0) {
          a.stats[token] = run_max[t];
          a.stats[N + token] = inv_sum;
        }
      }
    }
  };

  const int full = S / NBT;
  const int rem = S - full * NBT;
  for (int r = 0; r < full; ++r) {
#pragma unroll
    for (int j = 0; j < NB; ++j) step(j, r * NBT + j / T, true);
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (j / T < rem) step(j, full * NBT + j / T, false);
  }
}

// ----------------------------------------------------------------- backward

// What the backward needs per token besides the value rows: dO (packed BF16),
// the saved output and its refinement bytes (for delta = <dO, o>) and the
// softmax statistics.
template <int CH>
struct TokenRows {
  u32x4 g[CH];
  u32x4 o[CH];
  u32x2 r[CH];
  float run_max;
  float inv_sum;
};

template <int G, int CH, bool VEC, class Rows, class Grads>
__device__ __forceinline__ void load_token(const BwdArgs<Rows, Grads>& a, int64_t token, int lane,
                                           TokenRows<CH>& t) {
  const int D = a.width;
  load_row<G, CH, VEC>(a.grad_out + token * D, lane, D, t.g);
  load_row<G, CH, VEC>(a.out + token * D, lane, D, t.o);
  const int8_t* refine = a.out_refine + token * D;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    if constexpr (VEC) {
      t.r[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(refine + (d0 < D ? d0 : 0)));
    } else {
      uint32_t rq[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        const uint32_t b = static_cast<uint8_t>(refine[d0 + e < D ? d0 + e : D - 1]);
        rq[e >> 2] |= b << (8 * (e & 3));
      }
      t.r[c] = u32x2{rq[0], rq[1]};
    }
  }
  t.run_max = a.stats[token];
  t.inv_sum = a.stats[a.n_tokens + token];
}

// Low-order part of a refined output element: q * ulp(bf16)/256 (see
// refine_encode), exactly 0 when q == 0.
__device__ __forceinline__ float refine_delta(uint32_t bf16_bits, int q) {
  const int e = static_cast<int>((bf16_bits >> 7) & 0xffu);
  const float unit = __uint_as_float(static_cast<uint32_t>(min(max(e, 16), 254) - 15) << 23);
  return (e >= 16 && e <= 254) ? static_cast<float>(q) * unit : 0.0f;
}

// delta = <dO, o> over this lane's elements (dO already zero beyond D).  The
// BF16 part of o goes through the same dot2 sequence as dw = <v, dO>, and the
// refinement is added last: when o equals a source row exactly (one source,
// or identical sources) delta and dw are then bitwise equal and
// dz = p (dw - delta) is exactly zero, as in the oracle.
template <int CH>
__device__ __forceinline__ float token_delta(const TokenRows<CH>& t) {
  float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    m0 = dot2(t.o[c].x, t.g[c].x, m0);
    m1 = dot2(t.o[c].y, t.g[c].y, m1);
    m0 = dot2(t.o[c].z, t.g[c].z, m0);
    m1 = dot2(t.o[c].w, t.g[c].w, m1);
  }
  float corr = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const uint32_t w[4] = {t.o[c].x, t.o[c].y, t.o[c].z, t.o[c].w};
    const uint32_t gw[4] = {t.g[c].x, t.g[c].y, t.g[c].z, t.g[c].w};
    const uint32_t rq[2] = {t.r[c].x, t.r[c].y};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q0 = static_cast<int8_t>((rq[j >> 1] >> (16 * (j & 1))) & 0xffu);
      const int q1 = static_cast<int8_t>((rq[j >> 1] >> (16 * (j & 1) + 8)) & 0xffu);
      corr = fmaf(refine_delta(w[j] & 0xffffu, q0), bf16_lo(gw[j]), corr);
      corr = fmaf(refine_delta(w[j] >> 16, q1), bf16_hi(gw[j]), corr);
    }
  }
  return (m0 + m1) + corr;
}

// The query on this workgroup's row positions, FP32, +0 off the key (every
// group of the workgroup reads it from LDS).  Ends with a barrier.
template <int G, int CH>
__device__ __forceinline__ void fill_query_lds(const uint16_t* __restrict__ query, float* q_lds, int tail0, int D,
                                               int R) {
  for (int d = threadIdx.x; d < G * CH * kVec; d += kBlock) {
    const uint32_t bits = query[min(max(d - tail0, 0), R - 1)];
    q_lds[d] = (d >= tail0 && d < D) ? __uint_as_float(bits << 16) : 0.0f;
  }
  __syncthreads();
}

// Fixed-order reduction of the groups' dq into this block's partial row
// (`dq_lds` holds kBlock * kVec floats).  Every thread of the block calls it.
template <int G, int CH>
__device__ __forceinline__ void store_dq_partial(const float (&dq)[CH][kVec], float* dq_lds, float* partial,
                                                 int group, int lane, int tail0, int D) {
  constexpr int kGroups = kBlock / G;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
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

// One FP32 row (this lane's chunks, two 16-byte words each), unconditional
// like load_row: chunks at or beyond D read the row start (VEC) or clamped
// elements.  VEC requires 16-byte aligned rows and D % 8 == 0.
template <int G, int CH, bool VEC>
__device__ __forceinline__ void load_row_f32(const float* __restrict__ row, int lane, int D, u32x4 (&raw)[2 * CH]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int d0 = chunk_start<G>(c, lane);
    if constexpr (VEC) {
      const int at = d0 < D ? d0 : 0;
      raw[2 * c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + at));
      raw[2 * c + 1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + at + 4));
    } else {
      uint32_t w[kVec];
#pragma unroll
      for (int e = 0; e < kVec; ++e) w[e] = __float_as_uint(row[min(d0 + e, D - 1)]);
      raw[2 * c] = u32x4{w[0], w[1], w[2], w[3]};
      raw[2 * c + 1] = u32x4{w[4], w[5], w[6], w[7]};
    }
  }
}

// The gradient rows of one token seen as rows of width D (for prefetching the
// rows the accumulating backward adds to).
template <class Grads>
struct GradRows {
  const Grads& grad;
  int width;
  __device__ __forceinline__ const uint16_t* row(int s, int64_t n) const { return grad.row(s, n, width); }
};

// Persistent: group g takes tokens g, g + groups, ..., and the value rows
// stream through the ring across token boundaries.  The next token's dO,
// output, refinement bytes and statistics are requested `lead` = min(NB, S)
// items before the current token ends, right after a ring refill, and folded
// into delta on the token's last item -- when the younger rows in the ring
// are still in flight -- so a token switch does not drain the ring.
//
// ACC: the accumulating variant.  For a source whose bit is set in
// a.accumulate, the item's gradient row is prefetched with its value row (a
// second ring; other items load the idle row, so every load stays
// unconditional) and dv is stored as bf16(old + dv).
// With FP32 gradients (PackedGradsF32 / ListGradsF32: a source bank's sums)
// the rows are FP32: dv is written, or added, without BF16 rounding.
template <int G, int CH, int NB, bool NOMASK, bool VEC, bool ACC, class Rows, class Grads>
__global__ void __launch_bounds__(kBlock) attnres_bwd_kernel(const BwdArgs<Rows, Grads> a) {
  constexpr bool kF32 = kF32Grads<Grads>;
  constexpr bool kCoef = std::is_same_v<Grads, CoefSink>;
  static_assert(!kF32 || ACC, "FP32 gradient sums use the accumulating variant");
  static_assert(!kCoef || !ACC, "the coefficient backward writes no gradient rows");
  static_assert(G <= 64 || G == kBlock, "a wide group is the whole workgroup");
  constexpr int kGroups = kBlock / G;
  __shared__ float xred[xred_floats<G>(1)];
  __shared__ float dq_lds[kGroups * G * kVec];
  // The query on row positions, FP32, +0 off the key: read per item from LDS
  // (no registers; every group of the workgroup shares it).
  __shared__ __attribute__((aligned(16))) float q_lds[G * CH * kVec];
  const int lane = threadIdx.x % G;
  const int group = group_index<G>();
  const int D = a.width;
  const int R = a.rank;
  const int tail0 = D - R;
  const int S = a.n_sources;
  const float inv_R = 1.0f / static_cast<float>(R);
  const float scale = a.scale;
  int phase = 0;

  fill_query_lds<G, CH>(a.query, q_lds, tail0, D, R);
  uint32_t km[CH][4];
  if constexpr (!NOMASK) key_masks<G, CH>(lane, D, tail0, km);
  float dq[CH][kVec];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) dq[c][e] = 0.0f;

  // Group gid takes tokens gid, gid + groups, ...: at any time the groups
  // work on neighbouring tokens and walk the sources roughly in step, so the
  // rows in flight on the device lie in few, compact address ranges (row
  // blocks spread over the whole buffer are read and written measurably
  // slower).  Items are counted per group: first = 0, last = tokens * S.
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const int64_t groups = static_cast<int64_t>(gridDim.x) * kGroups;
  const int64_t my_tokens = gid < a.n_tokens ? (a.n_tokens - 1 - gid) / groups + 1 : 0;
  const int64_t first = 0;
  const int64_t last = my_tokens * S;

  if (first < last) {
    const int64_t last_token = gid + (my_tokens - 1) * groups;
    const int lead = NB < S ? NB : S;
    ItemCursor at{gid, 0, groups};

    // Current token state: dO (packed), delta and the softmax statistics.
    u32x4 g[CH];
    float delta, run_max, inv_sum;
    TokenRows<CH> pend;  // rows of the next token, between request and fold
    auto fold = [&]() __attribute__((always_inline)) {
      if constexpr (!NOMASK) mask_range<G, CH>(lane, D, pend.g);
      float red[1] = {token_delta<CH>(pend)};
      group_sum<G, 1>(red, xred, phase);
      delta = red[0];
#pragma unroll
      for (int c = 0; c < CH; ++c) g[c] = pend.g[c];
      run_max = pend.run_max;
      inv_sum = pend.inv_sum;
    };
    load_token<G, CH, VEC>(a, at.token, lane, pend);
    fold();
    __builtin_amdgcn_sched_barrier(0);
    // The second token's request point may lie before the range start.
    if (at.source > S - lead && at.token < last_token) load_token<G, CH, VEC>(a, at.token + groups, lane, pend);

    const uint16_t* idle = a.src.row(0, at.token);
    ItemCursor ahead = at;
    int64_t ahead_item = first;
    u32x4 ring[NB][CH];
    float ring_z[NB];
    float ring_r[NB];
    u32x4 ring_old[ACC ? NB : 1][kF32 ? 2 * CH : CH];  // ACC: the gradient rows dv is added to
    bool ring_acc[ACC ? NB : 1];
    auto refill_slot = [&](int j) __attribute__((always_inline)) {
      const bool live = ahead_item < last;
      refill<G, CH, VEC>(a.src, ahead, live, idle, lane, D, ring[j]);
      if constexpr (ACC) {
        ring_acc[j] = live && a.accumulates(ahead.source);
        if constexpr (kF32) {
          // idle: row (0, 0) of the FP32 buffer (always 4*D bytes, cache-resident)
          const float* row = ring_acc[j] ? a.grad.row(ahead.source, ahead.token, D) : a.grad.row(0, 0, D);
          load_row_f32<G, CH, VEC>(row, lane, D, ring_old[j]);
        } else {
          refill<G, CH, VEC>(GradRows<Grads>{a.grad, D}, ahead, ring_acc[j], idle, lane, D, ring_old[j]);
        }
      }
      const int64_t at_item = live ? ahead.token * S + ahead.source : 0;
      ring_z[j] = a.logit[at_item];
      ring_r[j] = a.inv_rms[at_item];
      if (live) {
        ++ahead_item;
        ahead.advance(S);
      }
    };
#pragma unroll
    for (int j = 0; j < NB; ++j) refill_slot(j);

    auto step = [&](int j, bool refill) __attribute__((always_inline)) {
      const int s = at.source;
      const int64_t token = at.token;
      float dw[1] = {0.0f};
      {
        float dw1 = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          dw[0] = dot2(ring[j][c].x, g[c].x, dw[0]);
          dw1 = dot2(ring[j][c].y, g[c].y, dw1);
          dw[0] = dot2(ring[j][c].z, g[c].z, dw[0]);
          dw1 = dot2(ring[j][c].w, g[c].w, dw1);
        }
        dw[0] += dw1;
      }
      group_sum<G, 1>(dw, xred, phase);
      const float z = ring_z[j];
      const float inv_rms = ring_r[j];
      const float p = __expf(z - run_max) * inv_sum;
      const float dz = p * (dw[0] - delta);
      const float ca = inv_rms * (dz * scale);                  // on q; dq += ca * key
      const float cb = -(inv_rms * inv_rms) * (dz * z * inv_R);  // on the key coordinates
      if constexpr (kCoef) {
        // coefficient backward: p, a, b for the later gather, dq here; no dv row
        if (lane == 0) {
          float* plane = a.grad.coef + static_cast<int64_t>(s) * a.n_tokens + token;
          const int64_t stride = static_cast<int64_t>(S) * a.n_tokens;
          plane[0] = p;
          plane[stride] = ca;
          plane[2 * stride] = cb;
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const uint32_t w[4] = {ring[j][c].x, ring[j][c].y, ring[j][c].z, ring[j][c].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t kw = NOMASK ? w[k] : (w[k] & km[c][k]);
            dq[c][2 * k] = fmaf(ca, bf16_lo(kw), dq[c][2 * k]);
            dq[c][2 * k + 1] = fmaf(ca, bf16_hi(kw), dq[c][2 * k + 1]);
          }
        }
      } else {
      auto* grad_row = a.grad.row(s, token, D);
      // dO is unpacked per item with a shift and mask the compiler cannot
      // prove loop-invariant (s >= 0, so both equal the constants): a hoisted
      // unpacked copy of dO would cost 32 registers per lane.
      const uint32_t lo_shift = 16u | (static_cast<uint32_t>(s) >> 31);
      const uint32_t hi_mask = 0xffff0000u | (static_cast<uint32_t>(s) >> 31);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int d0 = chunk_start<G>(c, lane);
        const uint32_t w[4] = {ring[j][c].x, ring[j][c].y, ring[j][c].z, ring[j][c].w};
        const uint32_t gw[4] = {g[c].x, g[c].y, g[c].z, g[c].w};
        const float4 qa = *reinterpret_cast<const float4*>(&q_lds[d0]);
        const float4 qb = *reinterpret_cast<const float4*>(&q_lds[d0 + 4]);
        const float qf[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t out[4];
        float outf[kF32 ? kVec : 1];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t kw = NOMASK ? w[k] : (w[k] & km[c][k]);
          const float k0 = bf16_lo(kw), k1 = bf16_hi(kw);
          const float g0 = __uint_as_float(gw[k] << lo_shift), g1 = __uint_as_float(gw[k] & hi_mask);
          float v0 = fmaf(cb, k0, fmaf(ca, qf[2 * k], p * g0));
          float v1 = fmaf(cb, k1, fmaf(ca, qf[2 * k + 1], p * g1));
          dq[c][2 * k] = fmaf(ca, k0, dq[c][2 * k]);
          dq[c][2 * k + 1] = fmaf(ca, k1, dq[c][2 * k + 1]);
          if constexpr (kF32) {
            const u32x4& ow = ring_old[j][2 * c + (k >> 1)];
            const uint32_t o0 = (k & 1) ? ow.z : ow.x, o1 = (k & 1) ? ow.w : ow.y;
            outf[2 * k] = (ring_acc[j] ? __uint_as_float(o0) : 0.0f) + v0;
            outf[2 * k + 1] = (ring_acc[j] ? __uint_as_float(o1) : 0.0f) + v1;
          } else {
            if constexpr (ACC) {
              const uint32_t ow[4] = {ring_old[j][c].x, ring_old[j][c].y, ring_old[j][c].z, ring_old[j][c].w};
              v0 = (ring_acc[j] ? bf16_lo(ow[k]) : 0.0f) + v0;
              v1 = (ring_acc[j] ? bf16_hi(ow[k]) : 0.0f) + v1;
            }
            out[k] = pack_bf16x2(v0, v1);
          }
        }
        if constexpr (kF32) {
          if constexpr (VEC) {
            if (NOMASK || d0 < D) {
              __builtin_nontemporal_store(f32x4{outf[0], outf[1], outf[2], outf[3]},
                                          reinterpret_cast<f32x4*>(grad_row + d0));
              __builtin_nontemporal_store(f32x4{outf[4], outf[5], outf[6], outf[7]},
                                          reinterpret_cast<f32x4*>(grad_row + d0 + 4));
            }
          } else {
#pragma unroll
            for (int e = 0; e < kVec; ++e) {
              if (d0 + e < D) grad_row[d0 + e] = outf[e];
            }
          }
        } else if (NOMASK || d0 < D) {
          store_chunk<G, VEC>(grad_row, d0, D, u32x4{out[0], out[1], out[2], out[3]});
        }
      }
      }  // kCoef

      if (refill) {
        __builtin_amdgcn_sched_barrier(0);  // refill the slot after its last use
        refill_slot(j);
      }
      if (token < last_token) {
        if (s == S - lead) load_token<G, CH, VEC>(a, token + groups, lane, pend);
        if (s == S - 1) fold();
      }
      at.advance(S);
    };

    // Full rounds refill every slot; the remainder only drains the ring (see
    // the forward kernel for why no exit test sits between slots).
    const int64_t items = last - first;
    const int64_t rounds = items / NB;
    const int rem = static_cast<int>(items - rounds * NB);
    for (int64_t r = 0; r < rounds; ++r) {
#pragma unroll
      for (int j = 0; j < NB; ++j) step(j, true);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < rem) step(j, false);
    }
  }

  store_dq_partial<G, CH>(dq, dq_lds, a.partial + static_cast<int64_t>(blockIdx.x) * R, group, lane, tail0, D);
}

// ---------------------------------------------------- backward, token blocks

// Token-block backward for 64-lane rows of 4 chunks (D = 2048, R = D): a
// group owns T consecutive tokens at a time (blocks b, b + groups, ... of a
// persistent grid) and walks their items source-major, (s, 0), (s, 1), ...,
// (s, T-1), (s + 1, 0), ...  Ring slot t serves token t, so the value rows a
// group has in flight, and the dv rows it stores one after another, are one
// source's rows of adjacent tokens: a contiguous span.  The streaming kernel
// instead keeps consecutive sources of one token in flight, rows a source
// stride apart, and how fast those move depends on where the buffers lie in
// physical memory: at c2 the streaming backward takes 602-660 us depending on
// the placement of values and gradients, this kernel 590-610 us under every
// placement measured.  Per-token arithmetic is the streaming kernel's (same
// sums in the same order), so the results are bit-identical.
//
// The next block's dO, output, refinement bytes and statistics are requested
// two sources before the block ends and folded into delta after its last
// item; slots wrap into the next block without draining.  With T = 4 the
// kernel needs more than 256 registers (AGPRs hold the rest) and runs one
// wave per SIMD: four rows in flight per wave.  T = 2 and 3 were slower
// (680 and 700 us at c2).  It takes unmasked rows only (R = D = 2048): masked
// instances spilled (224 bytes per lane).  Its timing is sensitive to code generation: a version
// with a few equivalent source edits (a named request step, a hoisted idle
// row) compiled to a kernel that took 670 us instead of 590 us at c2, so
// changes here are measured before they are kept.
template <int G, int CH, int T, bool VEC, class Rows, class Grads>
__global__ void __launch_bounds__(kBlock) attnres_bwd_block_kernel(const BwdArgs<Rows, Grads> a) {
  static_assert(G == 64, "one wavefront per token");
  static_assert(std::is_same_v<Grads, PackedGrads> || std::is_same_v<Grads, ListGrads>, "BF16 dv rows");
  constexpr int kGroups = kBlock / G;
  __shared__ float xred[1];
  __shared__ float dq_lds[kGroups * G * kVec];
  __shared__ __attribute__((aligned(16))) float q_lds[G * CH * kVec];
  const int lane = threadIdx.x % G;
  const int group = group_index<G>();
  const int D = a.width;
  const int R = a.rank;
  const int tail0 = D - R;
  const int S = a.n_sources;
  const int64_t N = a.n_tokens;
  const float inv_R = 1.0f / static_cast<float>(R);
  const float scale = a.scale;
  int phase = 0;

  fill_query_lds<G, CH>(a.query, q_lds, tail0, D, R);
  float dq[CH][kVec];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) dq[c][e] = 0.0f;

  const int64_t n_blocks = (N + T - 1) / T;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const int64_t groups = static_cast<int64_t>(gridDim.x) * kGroups;
  const int64_t my_blocks = gid < n_blocks ? (n_blocks - 1 - gid) / groups + 1 : 0;

  if (my_blocks > 0) {
    // tokens of block b (clamped: a token past N repeats token N-1 and stores nothing)
    auto token_of = [&](int64_t b, int t) __attribute__((always_inline)) {
      const int64_t n = b * T + t;
      return n < N ? n : N - 1;
    };
    int64_t blk = gid;
    const int64_t last_blk = gid + (my_blocks - 1) * groups;
    u32x4 g[T][CH];
    float delta[T], run_max[T], inv_sum[T];
    TokenRows<CH> pend[T];
    auto request = [&](int64_t b) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < T; ++t) load_token<G, CH, VEC>(a, token_of(b, t), lane, pend[t]);
    };
    auto fold = [&]() __attribute__((always_inline)) {
      float red[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        red[t] = token_delta<CH>(pend[t]);
      }
      group_sum<G, T>(red, xred, phase);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        delta[t] = red[t];
#pragma unroll
        for (int c = 0; c < CH; ++c) g[t][c] = pend[t].g[c];
        run_max[t] = pend[t].run_max;
        inv_sum[t] = pend[t].inv_sum;
      }
    };
    request(blk);
    fold();
    __builtin_amdgcn_sched_barrier(0);

    // ring slot t: the next row of token t of the current (or next) block
    u32x4 ring[T][CH];
    float ring_z[T], ring_r[T];
    auto refill = [&](int t, int s, int64_t b, bool live) __attribute__((always_inline)) {
      const int64_t n = token_of(b, t);
      const uint16_t* row = live ? a.src.row(s, n) : a.src.row(0, token_of(blk, 0));
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int d0 = chunk_start<G>(c, lane);
        const int offset = (live && d0 < D) ? d0 : 0;
        if constexpr (VEC) {
          ring[t][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + offset));
        }
      }
      if constexpr (!VEC) load_row<G, CH, VEC>(row, lane, D, ring[t]);
      const int64_t item = live ? n * S + s : 0;
      ring_z[t] = a.logit[item];
      ring_r[t] = a.inv_rms[item];
    };
#pragma unroll
    for (int t = 0; t < T; ++t) refill(t, 0, blk, true);

    int s = 0;
    for (;;) {
      // next row of every slot: source s + 1 of this block, or source 0 of the next block
      const bool wrap = s + 1 == S;
      const int64_t nb = wrap ? blk + groups : blk;
      const bool live_next = !wrap || blk < last_blk;
      if (s == S - 2 && blk < last_blk) request(blk + groups);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int64_t token = token_of(blk, t);
        const bool valid = blk * T + t < N;
        float dw[1] = {0.0f};
        {
          float dw1 = 0.0f;
#pragma unroll
          for (int c = 0; c < CH; ++c) {
            dw[0] = dot2(ring[t][c].x, g[t][c].x, dw[0]);
            dw1 = dot2(ring[t][c].y, g[t][c].y, dw1);
            dw[0] = dot2(ring[t][c].z, g[t][c].z, dw[0]);
            dw1 = dot2(ring[t][c].w, g[t][c].w, dw1);
          }
          dw[0] += dw1;
        }
        group_sum<G, 1>(dw, xred, phase);
        const float z = ring_z[t];
        const float inv_rms = ring_r[t];
        const float p = __expf(z - run_max[t]) * inv_sum[t];
        const float dz = valid ? p * (dw[0] - delta[t]) : 0.0f;
        const float ca = inv_rms * (dz * scale);
        const float cb = -(inv_rms * inv_rms) * (dz * z * inv_R);
        auto* grad_row = a.grad.row(s, token, D);
        const uint32_t lo_shift = 16u | (static_cast<uint32_t>(s) >> 31);
        const uint32_t hi_mask = 0xffff0000u | (static_cast<uint32_t>(s) >> 31);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int d0 = chunk_start<G>(c, lane);
          const uint32_t w[4] = {ring[t][c].x, ring[t][c].y, ring[t][c].z, ring[t][c].w};
          const uint32_t gw[4] = {g[t][c].x, g[t][c].y, g[t][c].z, g[t][c].w};
          const float4 qa = *reinterpret_cast<const float4*>(&q_lds[d0]);
          const float4 qb = *reinterpret_cast<const float4*>(&q_lds[d0 + 4]);
          const float qf[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
          uint32_t out[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float k0 = bf16_lo(w[k]), k1 = bf16_hi(w[k]);
            const float g0 = __uint_as_float(gw[k] << lo_shift), g1 = __uint_as_float(gw[k] & hi_mask);
            const float v0 = fmaf(cb, k0, fmaf(ca, qf[2 * k], p * g0));
            const float v1 = fmaf(cb, k1, fmaf(ca, qf[2 * k + 1], p * g1));
            dq[c][2 * k] = fmaf(ca, k0, dq[c][2 * k]);
            dq[c][2 * k + 1] = fmaf(ca, k1, dq[c][2 * k + 1]);
            out[k] = pack_bf16x2(v0, v1);
          }
          if (valid) store_chunk<G, VEC>(grad_row, d0, D, u32x4{out[0], out[1], out[2], out[3]});
        }
        __builtin_amdgcn_sched_barrier(0);  // refill the slot after its last use
        refill(t, wrap ? 0 : s + 1, nb, live_next);
      }
      if (wrap) {
        if (blk == last_blk) break;
        fold();
        blk += groups;
        s = 0;
      } else {
        ++s;
      }
    }
  }

  store_dq_partial<G, CH>(dq, dq_lds, a.partial + static_cast<int64_t>(blockIdx.x) * R, group, lane, tail0, D);
}

// ------------------------------------------------ backward, recompute policy

// For S <= kRecomputeMaxSources the forward stores no refinement and this
// backward reads neither the output nor its refinement: a group holds every
// value row of its token at once, and delta = <dO, o> = sum_s p_s <v_s, dO>
// comes from the dw_s = <v_s, dO> it needs anyway (o = sum_s p_s v_s),
// summed in source order.  Grid-stride over tokens on the persistent grid;
// the S + 1 rows of a token are requested together and occupancy hides
// their latency.  SM (>= S) rows are held; rows s >= S re-read row 0
// (cached) and are not used, so reads of few sources take a small SM.
template <int G, int CH, int SM, bool NOMASK, bool VEC, class Rows, class Grads>
__global__ void __launch_bounds__(kBlock) attnres_bwd_recompute_kernel(const BwdArgs<Rows, Grads> a) {
  static_assert(G <= 64 || G == kBlock, "a wide group is the whole workgroup");
  constexpr int kGroups = kBlock / G;
  __shared__ float xred[xred_floats<G>(SM)];
  __shared__ float dq_lds[kGroups * G * kVec];
  __shared__ __attribute__((aligned(16))) float q_lds[G * CH * kVec];
  const int lane = threadIdx.x % G;
  const int group = group_index<G>();
  const int D = a.width;
  const int R = a.rank;
  const int tail0 = D - R;
  const int S = a.n_sources;
  const float inv_R = 1.0f / static_cast<float>(R);
  const float scale = a.scale;
  int phase = 0;

  fill_query_lds<G, CH>(a.query, q_lds, tail0, D, R);
  uint32_t km[CH][4];
  if constexpr (!NOMASK) key_masks<G, CH>(lane, D, tail0, km);
  float dq[CH][kVec];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) dq[c][e] = 0.0f;

  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const int64_t groups = static_cast<int64_t>(gridDim.x) * kGroups;
  const int64_t my_tokens = gid < a.n_tokens ? (a.n_tokens - 1 - gid) / groups + 1 : 0;
  for (int64_t i = 0; i < my_tokens; ++i) {
    const int64_t token = gid + i * groups;
    u32x4 g[CH];
    u32x4 v[SM][CH];
    load_row<G, CH, VEC>(a.grad_out + token * D, lane, D, g);
#pragma unroll
    for (int s = 0; s < SM; ++s) load_row<G, CH, VEC>(a.src.row(s < S ? s : 0, token), lane, D, v[s]);
    float z[SM], ir[SM];
#pragma unroll
    for (int s = 0; s < SM; ++s) {
      const int64_t item = token * S + (s < S ? s : 0);
      z[s] = a.logit[item];
      ir[s] = a.inv_rms[item];
    }
    const float run_max = a.stats[token];
    const float inv_sum = a.stats[a.n_tokens + token];
    if constexpr (!NOMASK) mask_range<G, CH>(lane, D, g);

    float dw[SM];
#pragma unroll
    for (int s = 0; s < SM; ++s) {
      float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        d0 = dot2(v[s][c].x, g[c].x, d0);
        d1 = dot2(v[s][c].y, g[c].y, d1);
        d0 = dot2(v[s][c].z, g[c].z, d0);
        d1 = dot2(v[s][c].w, g[c].w, d1);
      }
      dw[s] = d0 + d1;
    }
    group_sum<G, SM>(dw, xred, phase);
    float p[SM];
    float delta = 0.0f;
#pragma unroll
    for (int s = 0; s < SM; ++s) {
      p[s] = __expf(z[s] - run_max) * inv_sum;
      delta = s < S ? fmaf(p[s], dw[s], delta) : delta;
    }

#pragma unroll
    for (int s = 0; s < SM; ++s) {
      if (s >= S) break;  // uniform
      const float dz = p[s] * (dw[s] - delta);
      const float ca = ir[s] * (dz * scale);                    // on q; dq += ca * key
      const float cb = -(ir[s] * ir[s]) * (dz * z[s] * inv_R);  // on the key coordinates
      uint16_t* grad_row = a.grad.row(s, token, D);
      // dO unpacked per source (see the streaming kernel: a hoisted unpacked
      // copy would cost CH * 8 registers).
      const uint32_t lo_shift = 16u | (static_cast<uint32_t>(s + S) >> 31);
      const uint32_t hi_mask = 0xffff0000u | (static_cast<uint32_t>(s + S) >> 31);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int d0 = chunk_start<G>(c, lane);
        const uint32_t w[4] = {v[s][c].x, v[s][c].y, v[s][c].z, v[s][c].w};
        const uint32_t gw[4] = {g[c].x, g[c].y, g[c].z, g[c].w};
        const float4 qa = *reinterpret_cast<const float4*>(&q_lds[d0]);
        const float4 qb = *reinterpret_cast<const float4*>(&q_lds[d0 + 4]);
        const float qf[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t out[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t kw = NOMASK ? w[k] : (w[k] & km[c][k]);
          const float k0 = bf16_lo(kw), k1 = bf16_hi(kw);
          const float g0 = __uint_as_float(gw[k] << lo_shift), g1 = __uint_as_float(gw[k] & hi_mask);
          const float v0 = fmaf(cb, k0, fmaf(ca, qf[2 * k], p[s] * g0));
          const float v1 = fmaf(cb, k1, fmaf(ca, qf[2 * k + 1], p[s] * g1));
          dq[c][2 * k] = fmaf(ca, k0, dq[c][2 * k]);
          dq[c][2 * k + 1] = fmaf(ca, k1, dq[c][2 * k + 1]);
          out[k] = pack_bf16x2(v0, v1);
        }
        if (NOMASK || d0 < D) store_chunk<G, VEC>(grad_row, d0, D, u32x4{out[0], out[1], out[2], out[3]});
      }
    }
  }
  store_dq_partial<G, CH>(dq, dq_lds, a.partial + static_cast<int64_t>(blockIdx.x) * R, group, lane, tail0, D);
}

// ------------------------------------------- backward, key-resident (R < D)

// For a read whose key is a suffix of whole chunk columns (D = G*CH*8,
// R = KC*G*8: KC = 1 or 2 of 4 or 8 columns, or the whole row of 4 columns,
// D = R = 2048) of at most KS sources, the forward stores no
// refinement and this backward reads neither the output nor its refinement,
// like the recompute kernel, but it streams the value rows through a ring
// instead of holding whole tokens.  Only the key coordinates of dv depend on
// delta:
//     dv_s = p_s dO  +  [key] (a_s q + b_s v_s),   a_s, b_s proportional to
//     dz_s = p_s (dw_s - delta),  delta = sum_s p_s dw_s.
// So each item stores the non-key part of its dv row (p_s dO) at once, adds
// p_s dw_s to delta (in source order, as the recompute kernel does) and keeps
// the key chunks of its value row in registers (KC chunks per source); after
// the token's last item, delta is complete and the key part of every dv row
// is formed from the held chunks.  The value rows are read once, the saved
// output never: the backward moves its algorithmic bytes, and delta is the
// exact FP32 sum instead of the refined BF16 output's.
//
// Group = one wavefront (G = 64).  Grid-stride over tokens like the streaming
// kernel; NB value rows in flight in a ring that crosses token boundaries.
// Items are counted per token with S rounded up to a multiple of NB (an item
// past S is padding and does nothing), so slot j always serves items
// j, j + NB, ... and every register index is a compile-time constant.  The
// next token's dO and statistics are requested two items before the token
// ends.
template <int G, int CH, int KC, int KS, int NB, bool LAG, bool VEC, class Rows, class Grads>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1)))
attnres_bwd_keyres_kernel(const BwdArgs<Rows, Grads> a) {
  static_assert(G == 64, "one wavefront per token group");
  static_assert(KC >= 1 && KC <= CH, "the key is a suffix of whole chunk columns");
  static_assert(KS % NB == 0, "whole ring rounds per token");
  static_assert(std::is_same_v<Grads, PackedGrads> || std::is_same_v<Grads, ListGrads>, "BF16 dv rows");
  constexpr int C0 = CH - KC;  // first key chunk column
  constexpr int kGroups = kBlock / G;
  __shared__ float dq_lds[kGroups * G * kVec];
  __shared__ __attribute__((aligned(16))) float q_lds[KC * G * kVec];
  const int lane = threadIdx.x % G;
  const int group = group_index<G>();
  const int D = a.width;  // G * CH * 8
  const int R = a.rank;   // KC * G * 8
  const int S = a.n_sources;
  const int Sp = (S + NB - 1) / NB * NB;
  const float inv_R = 1.0f / static_cast<float>(R);
  const float scale = a.scale;
  int phase = 0;

  for (int i = threadIdx.x; i < KC * G * kVec; i += kBlock) q_lds[i] = __uint_as_float(uint32_t{a.query[i]} << 16);
  __syncthreads();
  float dq[KC][kVec];
#pragma unroll
  for (int c = 0; c < KC; ++c)
#pragma unroll
    for (int e = 0; e < kVec; ++e) dq[c][e] = 0.0f;

  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const int64_t groups = static_cast<int64_t>(gridDim.x) * kGroups;
  const int64_t my_tokens = gid < a.n_tokens ? (a.n_tokens - 1 - gid) / groups + 1 : 0;

  if (my_tokens > 0) {
    int64_t token = gid;
    u32x4 g[CH], pend_g[CH];
    float run_max = a.stats[token], inv_sum = a.stats[a.n_tokens + token];
    float pend_max = run_max, pend_sum = inv_sum;
    load_row<G, CH, VEC>(a.grad_out + token * D, lane, D, g);
    // A padding item (past S, or past the group's last token) is never
    // consumed.  For 4096-wide rows it loads nothing (a uniform branch); for
    // 2048-wide rows it loads a row that is already cached: with a key of 2 or
    // 4 columns one row shared by every group, which stays in L2 (the group's
    // own first row is evicted between uses and re-read from HBM), with a key
    // of one column the group's first row, as measured fastest (see the
    // launcher).
    const uint16_t* idle = KC >= 2 ? a.src.row(0, 0) : a.src.row(0, token);
    u32x4 ring[NB][CH] = {};
    float ring_z[NB] = {}, ring_r[NB] = {};
    auto load_item = [&](int j, int64_t tok, int s, bool live) __attribute__((always_inline)) {
      if constexpr (CH == 8) {
        if (live) {
          load_row<G, CH, VEC>(a.src.row(s, tok), lane, D, ring[j]);
          ring_z[j] = a.logit[tok * S + s];
          ring_r[j] = a.inv_rms[tok * S + s];
        }
      } else {
        load_row<G, CH, VEC>(live ? a.src.row(s, tok) : idle, lane, D, ring[j]);
        const int64_t item = live ? tok * S + s : 0;
        ring_z[j] = a.logit[item];
        ring_r[j] = a.inv_rms[item];
      }
    };
#pragma unroll
    for (int j = 0; j < NB; ++j) load_item(j, token, j, j < S);

    // Held state of the previous token of the group: per source its key
    // chunks and scalars, and the key chunks of its dO and its delta.
    u32x4 key[KS][KC];
    float kp[KS], kdw[KS], kz[KS], kr[KS];
    constexpr int kHeldG = LAG ? CH : KC;  // chunks of the previous token's dO held: all, or the key's
    u32x4 gprev[kHeldG];
    float delta_prev = 0.0f;
    int64_t prev = -1;  // none yet

    // The key part of dv row (ss, prev) -- the previous token's delta is
    // complete -- and its dq terms.
    auto finish = [&](int ss) __attribute__((always_inline)) {
      const float p = kp[ss];
      const float dz = p * (kdw[ss] - delta_prev);
      const float ca = kr[ss] * (dz * scale);
      const float cb = -(kr[ss] * kr[ss]) * (dz * kz[ss] * inv_R);
      uint16_t* grad_row = a.grad.row(ss, prev, D);
      if constexpr (LAG) {  // the non-key part too: one whole-row store
#pragma unroll
        for (int c = 0; c < C0; ++c) {
          const uint32_t gw[4] = {gprev[c].x, gprev[c].y, gprev[c].z, gprev[c].w};
          uint32_t out[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) out[k] = pack_bf16x2(p * bf16_lo(gw[k]), p * bf16_hi(gw[k]));
          store_chunk<G, VEC>(grad_row, chunk_start<G>(c, lane), D, u32x4{out[0], out[1], out[2], out[3]});
        }
      }
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const uint32_t w[4] = {key[ss][c].x, key[ss][c].y, key[ss][c].z, key[ss][c].w};
        u32x4 gk;
        if constexpr (LAG) {
          gk = gprev[C0 + c];
        } else {
          gk = gprev[c];
        }
        const uint32_t gw[4] = {gk.x, gk.y, gk.z, gk.w};
        const float4 qa = *reinterpret_cast<const float4*>(&q_lds[(c * G + lane) * kVec]);
        const float4 qb = *reinterpret_cast<const float4*>(&q_lds[(c * G + lane) * kVec + 4]);
        const float qf[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t out[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float k0 = bf16_lo(w[k]), k1 = bf16_hi(w[k]);
          const float v0 = fmaf(cb, k0, fmaf(ca, qf[2 * k], p * bf16_lo(gw[k])));
          const float v1 = fmaf(cb, k1, fmaf(ca, qf[2 * k + 1], p * bf16_hi(gw[k])));
          dq[c][2 * k] = fmaf(ca, k0, dq[c][2 * k]);
          dq[c][2 * k + 1] = fmaf(ca, k1, dq[c][2 * k + 1]);
          out[k] = pack_bf16x2(v0, v1);
        }
        store_chunk<G, VEC>(grad_row, chunk_start<G>(C0 + c, lane), D, u32x4{out[0], out[1], out[2], out[3]});
      }
    };

    // Item ss of a token also finishes source ss of the group's previous
    // token (both have S items), so the key-part work is spread over the
    // stream instead of bunching at each token's end.  4096-wide rows do that
    // first, before the item's own dot product (the row stores and their
    // arithmetic then overlap the wait for the item's row); 2048-wide rows
    // after the slot's refill.  Measured on MI355X (backward us, after ->
    // first): c3 798.8 -> 771.5; S = 9, D = 4096, R = 1024: 459.4 -> 446.0;
    // S = 13, R = 512: 655.0 -> 647.8; but c4's shape 465.1 -> 511.0 and
    // S = 12, D = R = 2048 300.0 -> 320.6.  Results are identical: only
    // independent work moves, and dq accumulates in the same order.
    constexpr bool kFinishFirst = CH == 8;
    for (int64_t ti = 0; ti < my_tokens; ++ti) {
      const bool more = ti + 1 < my_tokens;
      const int64_t next = token + groups;
      const int request_at = S > 2 ? S - 2 : 0;
      float delta = 0.0f;
#pragma unroll
      for (int ss = 0; ss < KS; ++ss) {
        if (ss >= Sp) continue;  // uniform; a constant trip count keeps every register index static
        const int j = ss % NB;
        float p = 0.0f, dw[1] = {0.0f};
        u32x4 held[KC];
        if constexpr (kFinishFirst) {
          if (ss < S && prev >= 0) finish(ss);  // uniform
        }
        if (ss < S) {
          {
            float dw1 = 0.0f;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
              dw[0] = dot2(ring[j][c].x, g[c].x, dw[0]);
              dw1 = dot2(ring[j][c].y, g[c].y, dw1);
              dw[0] = dot2(ring[j][c].z, g[c].z, dw[0]);
              dw1 = dot2(ring[j][c].w, g[c].w, dw1);
            }
            dw[0] += dw1;
          }
          group_sum<G, 1>(dw, nullptr, phase);  // G = 64: wavefront sums, no LDS
          p = __expf(ring_z[j] - run_max) * inv_sum;
          delta = fmaf(p, dw[0], delta);
          if constexpr (!LAG) {  // the non-key part of this item's dv row now
            uint16_t* grad_row = a.grad.row(ss, token, D);
#pragma unroll
            for (int c = 0; c < C0; ++c) {
              const uint32_t gw[4] = {g[c].x, g[c].y, g[c].z, g[c].w};
              uint32_t out[4];
#pragma unroll
              for (int k = 0; k < 4; ++k) out[k] = pack_bf16x2(p * bf16_lo(gw[k]), p * bf16_hi(gw[k]));
              store_chunk<G, VEC>(grad_row, chunk_start<G>(c, lane), D, u32x4{out[0], out[1], out[2], out[3]});
            }
          }
#pragma unroll
          for (int c = 0; c < KC; ++c) held[c] = ring[j][C0 + c];
        }
        const float z_now = ring_z[j], r_now = ring_r[j];  // the refill below replaces them
        if (more && ss == request_at) {
          load_row<G, CH, VEC>(a.grad_out + next * D, lane, D, pend_g);
          pend_max = a.stats[next];
          pend_sum = a.stats[a.n_tokens + next];
        }
        __builtin_amdgcn_sched_barrier(0);  // refill the slot after its last use
        const int sn = ss + NB;
        if (sn < Sp) {
          load_item(j, token, sn, sn < S);
        } else {
          load_item(j, next, sn - Sp, more && sn - Sp < S);
        }
        if (ss < S) {
          if constexpr (!kFinishFirst) {
            if (prev >= 0) finish(ss);  // uniform
          }
#pragma unroll
          for (int c = 0; c < KC; ++c) key[ss][c] = held[c];
          kp[ss] = p;
          kdw[ss] = dw[0];
          kz[ss] = z_now;
          kr[ss] = r_now;
        }
      }
      delta_prev = delta;
#pragma unroll
      for (int c = 0; c < kHeldG; ++c) gprev[c] = g[LAG ? c : C0 + c];
      prev = token;
      if (more) {
#pragma unroll
        for (int c = 0; c < CH; ++c) g[c] = pend_g[c];
        run_max = pend_max;
        inv_sum = pend_sum;
      }
      token = next;
    }
#pragma unroll
    for (int ss = 0; ss < KS; ++ss) {
      if (ss < S) finish(ss);  // the group's last token
    }
  }

  // this block's dq partial row (key coordinates only; R = KC * G * 8), the
  // groups summed in a fixed order
  float* partial = a.partial + static_cast<int64_t>(blockIdx.x) * R;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
#pragma unroll
    for (int e = 0; e < kVec; ++e) dq_lds[group * (G * kVec) + lane * kVec + e] = dq[c][e];
    __syncthreads();
    for (int j = threadIdx.x; j < G * kVec; j += kBlock) {
      float t = dq_lds[j];
#pragma unroll
      for (int k = 1; k < kGroups; ++k) t += dq_lds[k * (G * kVec) + j];
      partial[c * G * kVec + j] = t;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------- source-bank gather

// The gradient of one source-bank slot, gathered from the reads that saw it:
//   grad[n] = sum_r ( p_r dO_r[n] + a_r q_r ) + [key] (sum_r b_r) v[n]
// with p, a, b of read r at token n as its coefficient backward wrote them --
// the same terms as the read's own dv, summed over the reads in FP32 in one
// pass instead of one read-modify-write of an FP32 sum per read.  The reads
// of a launch share R, so the b terms meet in one scalar per token.
// A group takes T consecutive tokens at a time (grid-stride over token
// blocks), so each read's query row is loaded once per T tokens and its
// coefficients for the T tokens are contiguous.  A ring of RING reads keeps
// the next reads' rows in flight while one is added.
// BF16OUT: the sums are stored rounded to BF16 (round to nearest even), for a
// BF16 source, instead of an FP32 row converted by a separate pass.
template <int G, int CH, bool VEC, bool BF16OUT, int RING>
__global__ void __launch_bounds__(kBlock) attnres_gather_kernel(const GatherArgs a) {
  static_assert(kBlock % G == 0 && (G <= 64 || G % 64 == 0), "groups of whole wavefronts above 64 lanes");
  constexpr int T = CH >= 4 ? 1 : 4 / CH;      // tokens per group iteration
  constexpr int kRing = RING;                  // reads in flight per group (T rows each)
  constexpr int kGroups = kBlock / G;
  const int lane = threadIdx.x % G;
  const int group = group_index<G>();
  const int D = a.width;
  const int64_t N = a.n_tokens;
  const int n_reads = a.n_reads;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroups + group;
  const int64_t groups = static_cast<int64_t>(gridDim.x) * kGroups;
  const int64_t blocks = (N + T - 1) / T;
  for (int64_t blk = gid; blk < blocks; blk += groups) {
    const int64_t token0 = blk * T;
    int64_t tok[T];  // clamped: a block past N re-reads the last token and stores nothing for it
#pragma unroll
    for (int t = 0; t < T; ++t) tok[t] = token0 + t < N ? token0 + t : N - 1;
    float acc[T][CH][kVec];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[t][c][e] = 0.0f;
    float bsum[T];
#pragma unroll
    for (int t = 0; t < T; ++t) bsum[t] = 0.0f;
    u32x4 g[kRing][T][CH], q[kRing][CH];
    float cp[kRing][T], ca[kRing][T], cb[kRing][T];
    auto request = [&](int b, int r) __attribute__((always_inline)) {
      const GatherRead& rd = a.read[r < n_reads ? r : n_reads - 1];  // past the end: the last read again
      load_row<G, CH, VEC>(rd.qrow, lane, D, q[b]);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        load_row<G, CH, VEC>(rd.grad_out + tok[t] * D, lane, D, g[b][t]);
        cp[b][t] = rd.p[tok[t]];
        ca[b][t] = rd.p[rd.plane_stride + tok[t]];
        cb[b][t] = rd.p[2 * rd.plane_stride + tok[t]];
      }
    };
    auto add = [&](int b) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        bsum[t] += cb[b][t];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const uint32_t gw[4] = {g[b][t][c].x, g[b][t][c].y, g[b][t][c].z, g[b][t][c].w};
          const uint32_t qw[4] = {q[b][c].x, q[b][c].y, q[b][c].z, q[b][c].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            acc[t][c][2 * k] = fmaf(ca[b][t], bf16_lo(qw[k]), fmaf(cp[b][t], bf16_lo(gw[k]), acc[t][c][2 * k]));
            acc[t][c][2 * k + 1] =
                fmaf(ca[b][t], bf16_hi(qw[k]), fmaf(cp[b][t], bf16_hi(gw[k]), acc[t][c][2 * k + 1]));
          }
        }
      }
    };
#pragma unroll
    for (int j = 0; j < kRing; ++j) request(j, j);
    for (int r = 0; r < n_reads; r += kRing) {
#pragma unroll
      for (int j = 0; j < kRing; ++j) {
        if (r + j < n_reads) add(j);        // uniform
        __builtin_amdgcn_sched_barrier(0);  // refill the slot after its use
        request(j, r + j + kRing);
      }
    }
    // the key terms, then the earlier sum (accumulate) and the store
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (token0 + t >= N) break;  // uniform
      u32x4 v[CH];
      load_row<G, CH, VEC>(a.values + tok[t] * a.row_stride, lane, D, v);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int d0 = chunk_start<G>(c, lane);
        const uint32_t vw[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int d = d0 + 2 * k;
          acc[t][c][2 * k] = fmaf(d >= a.tail0 ? bsum[t] : 0.0f, bf16_lo(vw[k]), acc[t][c][2 * k]);
          acc[t][c][2 * k + 1] = fmaf(d + 1 >= a.tail0 ? bsum[t] : 0.0f, bf16_hi(vw[k]), acc[t][c][2 * k + 1]);
        }
        if constexpr (BF16OUT) {
          uint16_t* grad_row = static_cast<uint16_t*>(a.grad) + tok[t] * D;
          const u32x4 packed{pack_bf16x2(acc[t][c][0], acc[t][c][1]), pack_bf16x2(acc[t][c][2], acc[t][c][3]),
                             pack_bf16x2(acc[t][c][4], acc[t][c][5]), pack_bf16x2(acc[t][c][6], acc[t][c][7])};
          if (d0 < D) store_chunk<G, VEC>(grad_row, d0, D, packed);
          continue;
        }
        float* grad_row = static_cast<float*>(a.grad) + tok[t] * D;
        if (a.accumulate) {  // uniform
#pragma unroll
          for (int e = 0; e < kVec; ++e) acc[t][c][e] += grad_row[min(d0 + e, D - 1)];
        }
        if constexpr (VEC) {
          if (d0 < D) {
            __builtin_nontemporal_store(f32x4{acc[t][c][0], acc[t][c][1], acc[t][c][2], acc[t][c][3]},
                                        reinterpret_cast<f32x4*>(grad_row + d0));
            __builtin_nontemporal_store(f32x4{acc[t][c][4], acc[t][c][5], acc[t][c][6], acc[t][c][7]},
                                        reinterpret_cast<f32x4*>(grad_row + d0 + 4));
          }
        } else {
#pragma unroll
          for (int e = 0; e < kVec; ++e) {
            if (d0 + e < D) grad_row[d0 + e] = acc[t][c][e];
          }
        }
      }
    }
  }
}

// ----------------------------------------------------------------- launchers

// Ring depth (rows in flight per group) for a chunk count.  Measured on
// MI355X at S=25, D=2048: the forward is equally fast with 3 or 4 rows in
// flight (2 is slower).
template <int CH>
constexpr int fwd_ring() { return CH <= 4 ? 4 : 2; }

// Compute units of the current device (cached per device; 0 if unknown).
inline int64_t device_cus() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 0;
  static thread_local int cached_device = -1;
  static thread_local int64_t cached = 0;
  if (cached_device == device) return cached;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  cached_device = device;
  cached = cus;
  return cached;
}

// Backward ring depth.  One row per group, except two for aligned,
// non-accumulating rows of 4 chunks (the variants that keep two rows without
// spilling): at 64 lanes (D <= 2048) and 256 lanes (D > 4096) always, at
// 32 lanes (D <= 1024) when the grid holds at most 4 wavefronts per CU, where
// a group has a long chain of items and little else hides its latency.
// Measured on MI355X (backward, median of 8 interleaved rounds, us):
// S=25, N=16384, D=2048: 645 -> 637; S=9, N=8192, D=8192: 492 -> 483;
// S=25, N=2048, D=1024: 54 -> 47 (R=D), 55 -> 48 (R=256); but at N=16384,
// D=1024 two rows are 0.8% slower (occupancy 2 either way), and the
// accumulating and element-wise variants spill with two.  Rows of 8 chunks
// (64 lanes, D <= 4096) keep two rows without spilling only unmasked, and
// are 2-3% slower with them (S=25, N=16384, D=R=4096: 1273 -> 1316; with the
// iterative-minreg scheduler of the (64, 8) backward unit too: S=25 1295.5 ->
// 1329.5, S=13 715.1 -> 727.6, S=48 2487.9 -> 2514.9).
template <int CH, bool VEC, bool ACC>
constexpr bool kBwdTwoRowVariant = CH == 4 && VEC && !ACC;

// At most 4 wavefronts per CU for N tokens of G lanes each.
inline bool few_waves(int64_t n_tokens, int G) {
  const int64_t cus = device_cus();
  return cus > 0 && n_tokens * G <= 4 * 64 * cus;
}

// Workgroups of `Kernel` resident on the current device (cached per kernel
// and device; 0 if the runtime cannot tell).  The kernel is a template
// argument so that every instantiation has its own cache.
template <auto Kernel>
int64_t resident_blocks() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 0;
  static thread_local int cached_device = -1;
  static thread_local int64_t cached = 0;
  if (cached_device == device) return cached;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(Kernel), kBlock, 0) !=
          hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  cached_device = device;
  cached = static_cast<int64_t>(cus) * per_cu;
  return cached;
}

// Grid shape of the forward.  Many sources: one token per group --
// workgroups that start as others retire spread the output stores over time
// (a persistent grid, whose groups all finish a token at once, is 2-6%
// slower from S ~ 17 on).  Few sources: a persistent grid, whose groups
// stream the rows of consecutive tokens through the ring without draining it
// -- one token per group leaves a group only S rows to keep in flight before
// it retires.  Measured on MI355X at N = 16384 (8192 for D = 8192), forward
// time one token per group -> persistent: S = 1: 28 -> 26 us (D = 1024),
// 59 -> 40 (2048), 144 -> 72 (4096), 110 -> 68 (8192); S = 5: 52 -> 46 (1024),
// 98 -> 83 (2048), 227 -> 155 (4096); S = 9: 132 -> 126 (2048), 293 -> 241
// (4096), 262 -> 249 (8192); S = 13 at D = 2048: equal; S = 17: 216 -> 224.
constexpr int kPersistentFwdMaxSources = 12;

template <int G, int CH, int T, int NBT, bool NOMASK, bool VEC, class Rows>
void launch_fwd_block(const FwdArgs<Rows>& a, hipStream_t stream) {
  constexpr int64_t kTok = (kBlock / G) * T;
  const int64_t blocks = (a.n_tokens + kTok - 1) / kTok;
  hipLaunchKernelGGL((attnres_fwd_block_kernel<G, CH, T, NBT, NOMASK, VEC, Rows>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kBlock), 0, stream, a);
}

// Token blocks for few sources at D = R = 2048 (aligned, unmasked): two tokens
// per wavefront, two rows of each in flight, one block per group.  Measured on
// MI355X (forward alone, us, persistent one-token ring -> token blocks):
// S = 9, N = 32768: 252.7 -> 234.6; S = 12, N = 16384: 161.8 -> 152.7; S = 5,
// N = 32768: 157.9 -> 153.4.  Four tokens of one row each were slower at these
// S (254.6, 159.8, 176.0), and at D = 1024 (32-lane groups) the same change
// was mixed (S = 9: 123.8 -> 118.7; S = 12, R = 256: 78.4 -> 80.1).
constexpr int kFwdBlockMinSources = 5;

// Many sources at D = R = 2048: four tokens per wavefront, one row of each in
// flight (one wave per SIMD).  Measured on MI355X (forward alone, us, one token
// per group -> four), after a forward / after a backward of other values:
// S = 25, N = 16384: 319.6 -> 318.4 / 320.6 -> 299.8; S = 49, N = 8192:
// 298.4 -> 260.4 / 298.0 -> 261.5; but S = 16: 202.0 -> 199.3 / 202.8 -> 205.4.
// Right after the backward of the same values (a benchmark loop repeating one
// read) the one-token forward reads part of them from the memory-side cache and
// is as fast or faster (S = 25: 286.6 against 288.8).
constexpr int kFwdBlock4MinSources = 24;

// 64 lanes of 8 chunks (2048 < D <= 4096, 16-byte aligned rows), masked or
// not, past the persistent range: two tokens per wavefront, one row of each
// in flight.  Measured on MI355X (forward alone, N = 16384, us, one token per
// group -> token blocks): D = 3072, R = D: S = 13: 336 -> 264, S = 25: 540 ->
// 441, S = 48: 961 -> 797; D = 2560, R = 640: S = 25: 506 -> 404; D = R =
// 4096: S = 13: 361 -> 331, S = 25: 601 -> 588, S = 48: 1061 -> 1064; D =
// 4096, R = 1024: S = 13: 351 -> 327, S = 25: 601 -> 586, S = 48: 1059 ->
// 1067.  Rows of fewer than 4096 elements leave some chunks of a one-token
// group idle, and two tokens per wavefront keep more bytes in flight.  In the
// persistent range (S <= 12) the one-token ring stays: S = 5: 135 -> 153
// (D = 3072); two rows per token were slower everywhere.
template <int G, int CH, bool VEC>
constexpr bool kFwdBlock8Variant = G == 64 && CH == 8 && VEC;

// 64 lanes of 4 chunks with rows shorter than 2048 (1024 < D < 2048, aligned,
// so some chunks of a group idle), from kFwdBlockMinSources sources: the same
// two tokens per wavefront, one row of each in flight.  Measured on MI355X
// (forward alone, N = 16384, us, current -> token blocks): D = 1280, R = D:
// S = 5: 61.9 -> 58.8, S = 13: 137.4 -> 109.2, S = 48: 388.3 -> 343.2;
// D = 1536, R = D: S = 9: 100.7 -> 92.7, S = 13: 146.4 -> 124.7, S = 25:
// 241.6 -> 229.9, S = 48: 425.1 -> 429.3; R = 384: S = 13: 140.4 -> 124.6.
// Full rows of 2048 with key masks were mixed (R = 512: S = 13: 166.0 ->
// 170.0, S = 48: 635.6 -> 570.0) and keep the one-token kernel.
template <int G, int CH, bool NOMASK, bool VEC>
constexpr bool kFwdBlockShortVariant = G == 64 && CH == 4 && !NOMASK && VEC;

// Workgroup-wide token groups (256 lanes of 4 chunks, 4096 < D <= 8192,
// aligned), from kFwdBlockMinSources sources: two tokens per workgroup, one
// row of each in flight.  Measured on MI355X (forward alone, N = 8192, us,
// one token -> token blocks): D = 5120, R = D: S = 5: 120.1 -> 107.4, S = 25:
// 487.7 -> 374.4, S = 48: 872.9 -> 700.9; D = 6144, R = 1536: S = 25: 493.1 ->
// 452.8; D = 7168, R = D: S = 9: 228.6 -> 211.0; D = R = 8192: S = 9: 247.5 ->
// 239.4, S = 48: 1160.8 -> 1134.0; R = 2048: S = 25: 615.3 -> 622.0.  Two
// rows per token were slower than one.
template <int G, int CH, bool VEC>
constexpr bool kFwdBlockWideVariant = G == kBlock && CH == 4 && VEC;

// 32-lane token groups (two per wavefront), aligned rows: at 1 or 2 chunks per
// lane (128 < D <= 512) from kFwdBlockMinSources sources, two tokens per group
// with two rows of each in flight; at 4 chunks (512 < D < 1024, some idle) from
// kFwdBlockShort32MinSources, one row of each.  Measured on MI355X (forward
// alone, N = 16384, us, one token -> token blocks): D = 512, R = D: S = 5:
// 28.3 -> 23.3, S = 25: 85.2 -> 77.7, S = 48: 153.2 -> 146.3; D = 384: S = 9:
// 38.0 -> 30.8, S = 25: 83.0 -> 64.6, S = 48: 140.3 -> 126.2; D = 768, R = D:
// S = 9: 53.7 -> 53.0, S = 25: 125.1 -> 111.4, S = 48: 214.1 -> 200.6; D =
// 640, R = 160: S = 25: 115.1 -> 101.5; but S = 5: 37.2 -> 38.9 (D = 768);
// D = 256 (1 chunk): S = 9: 24.8 -> 23.4, S = 25: 51.2 -> 45.8; D = 200: S =
// 48: 86.6 -> 79.8.  Full rows of 1024 were within +-3% either way and keep
// the one-token kernel (a wavefront per token instead, 64 lanes of 2 chunks,
// four or eight tokens, was slower: S = 25, N = 16384, R = D: 153 -> 165-172,
// S = 48: 282-290 -> 292-309; S = 13 equal), as do 16-lane groups (D <= 128: within +-1.5%) and
// rows that are not 16-byte aligned (D = 3000, 1000, 5000: within +-1%).
template <int G, int CH, bool VEC>
constexpr bool kFwdBlock32NarrowVariant = G == 32 && CH <= 2 && VEC;
template <int G, int CH, bool NOMASK, bool VEC>
constexpr bool kFwdBlock32x4Variant = G == 32 && CH == 4 && !NOMASK && VEC;
constexpr int kFwdBlockShort32MinSources = 9;

template <int G, int CH, bool NOMASK, bool VEC, class Rows>
void launch_fwd(const FwdArgs<Rows>& a, hipStream_t stream) {
  constexpr int64_t kGroups = kBlock / G;
  if constexpr (G == 64 && CH == 4 && NOMASK && VEC) {
    if (a.n_sources >= kFwdBlockMinSources && a.n_sources <= kPersistentFwdMaxSources) {
      return launch_fwd_block<G, CH, 2, 2, NOMASK, VEC>(a, stream);
    }
    if (a.n_sources >= kFwdBlock4MinSources) return launch_fwd_block<G, CH, 4, 1, NOMASK, VEC>(a, stream);
  }
  if constexpr (kFwdBlock8Variant<G, CH, VEC>) {
    if (a.n_sources > kPersistentFwdMaxSources) return launch_fwd_block<G, CH, 2, 1, NOMASK, VEC>(a, stream);
  }
  if constexpr (kFwdBlockWideVariant<G, CH, VEC>) {
    if (a.n_sources >= kFwdBlockMinSources) return launch_fwd_block<G, CH, 2, 1, NOMASK, VEC>(a, stream);
  }
  if constexpr (kFwdBlock32NarrowVariant<G, CH, VEC>) {
    if (a.n_sources >= kFwdBlockMinSources) return launch_fwd_block<G, CH, 2, 2, NOMASK, VEC>(a, stream);
  }
  if constexpr (kFwdBlock32x4Variant<G, CH, NOMASK, VEC>) {
    if (a.n_sources >= kFwdBlockShort32MinSources && a.width < G * CH * kVec) {
      return launch_fwd_block<G, CH, 2, 1, NOMASK, VEC>(a, stream);
    }
  }
  if constexpr (kFwdBlockShortVariant<G, CH, NOMASK, VEC>) {
    if (a.n_sources >= kFwdBlockMinSources && a.width < G * CH * kVec) {
      return launch_fwd_block<G, CH, 2, 1, NOMASK, VEC>(a, stream);
    }
  }
  int64_t blocks = (a.n_tokens + kGroups - 1) / kGroups;
  if (a.n_sources <= kPersistentFwdMaxSources) {
    blocks = grid_blocks(a.n_tokens, G, resident_blocks<&attnres_fwd_kernel<G, CH, fwd_ring<CH>(), NOMASK, VEC, Rows>>());
  }
  hipLaunchKernelGGL((attnres_fwd_kernel<G, CH, fwd_ring<CH>(), NOMASK, VEC, Rows>),
                     dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream, a);
}

// The masked forwards of the (64, 8) geometry (2048 < D <= 4096, R < D) are
// compiled with that geometry's backward launchers (ATTNRES_UNIT_PART 2, the
// iterative-minreg machine scheduler); part 1 only declares them.  Measured on
// MI355X (forward alone, N = 16384, R = 1024, us, three rounds, default ->
// minreg): S = 16 381.1 / 390.5 / 377.3 -> 371.0 / 385.9 / 368.9; S = 13
// 309.1 / 307.8 / 308.2 -> 305.8 / 304.6 / 306.0; S = 25 566.6 / 568.8 /
// 571.0 -> 556.5 / 561.2 / 564.3; S = 48 1044.7 / 1039.0 / 1047.6 -> 1024.3 /
// 1026.9 / 1023.5.  The unmasked ones (R = D) were slower with it (S = 16:
// 388.5 / 392.0 / 386.2 -> 400.1 / 395.7 / 396.2) and stay in part 1.
#if defined(ATTNRES_LANES) && defined(ATTNRES_CHUNKS) && ATTNRES_LANES == 64 && ATTNRES_CHUNKS == 8 && \
    defined(ATTNRES_UNIT_PART) && ATTNRES_UNIT_PART == 1
extern template void launch_fwd<64, 8, false, true, PackedRows>(const FwdArgs<PackedRows>&, hipStream_t);
extern template void launch_fwd<64, 8, false, false, PackedRows>(const FwdArgs<PackedRows>&, hipStream_t);
extern template void launch_fwd<64, 8, false, true, ListRows>(const FwdArgs<ListRows>&, hipStream_t);
extern template void launch_fwd<64, 8, false, false, ListRows>(const FwdArgs<ListRows>&, hipStream_t);
#endif

template <int G, int CH, class Rows>
void launch_fwd_geometry(const FwdArgs<Rows>& a, bool nomask, bool vec, hipStream_t stream) {
  if (nomask) {
    if (vec) launch_fwd<G, CH, true, true>(a, stream);
    else launch_fwd<G, CH, true, false>(a, stream);
  } else {
    if (vec) launch_fwd<G, CH, false, true>(a, stream);
    else launch_fwd<G, CH, false, false>(a, stream);
  }
}

// The streaming backward's grid: up to two times the workgroups that fit on
// the device at once.  Its token shares are static, so with one resident
// grid the slowest workgroup sets the kernel's end (per-launch durations at
// c2 ranged 578-708 us on one box); with more, shorter workgroups the
// hardware hands the later ones to whichever CU frees up first.  Each
// workgroup also writes one dq partial row, which the reduction reads.
// Measured on MI355X (backward op, us): one resident grid -> two: c2 629 ->
// 617-624, c3 833 -> 827-829; two -> four on another box: c2 618 -> 627, c3
// 824 -> 826, c4 481 -> 486 (four: 2048 partial rows, a reduction of 11 us).
constexpr int64_t kBwdGridPerResident = 2;

template <int G, int CH, int NB, bool NOMASK, bool VEC, bool ACC, class Rows, class Grads>
int64_t launch_bwd_ring(const BwdArgs<Rows, Grads>& a, hipStream_t stream) {
  const int64_t resident = resident_blocks<&attnres_bwd_kernel<G, CH, NB, NOMASK, VEC, ACC, Rows, Grads>>();
  const int64_t blocks = grid_blocks(a.n_tokens, G, kBwdGridPerResident * resident, a.max_grid);
  hipLaunchKernelGGL((attnres_bwd_kernel<G, CH, NB, NOMASK, VEC, ACC, Rows, Grads>),
                     dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream, a);
  return blocks;
}

// The token-block backward (attnres_bwd_block_kernel) takes the plain
// backward of aligned, unmasked rows of 2048 elements (R = D) with BF16
// gradient rows, packed or list, T = 4 tokens per group, for reads of at
// least kBwdBlockMinSources sources.  Measured on MI355X (backward alone,
// us, streaming -> token blocks): S = 25, N = 16384: 602-670 -> 590-600;
// S = 13, N = 32768: 706-714 -> 656-668; S = 49, N = 8192: 610-635 -> 565;
// but S = 12, N = 16384: 309-312 -> 315; S = 9, N = 32768: 479-487 ->
// 501-516; S = 7: 390 -> 397-402 (fewer sources per block leave less to
// stream between the block switches).
template <int G, int CH, bool NOMASK, bool VEC, bool ACC, class Grads>
constexpr bool kBwdBlockVariant = G == 64 && CH == 4 && NOMASK && VEC && !ACC &&
                                  (std::is_same_v<Grads, PackedGrads> || std::is_same_v<Grads, ListGrads>);
constexpr int kBwdBlockTokens = 4;
constexpr int kBwdBlockMinSources = 13;

template <int G, int CH, int T, bool VEC, class Rows, class Grads>
int64_t launch_bwd_block(const BwdArgs<Rows, Grads>& a, hipStream_t stream) {
  const int64_t resident = resident_blocks<&attnres_bwd_block_kernel<G, CH, T, VEC, Rows, Grads>>();
  const int64_t blocks = grid_blocks((a.n_tokens + T - 1) / T, G, kBwdGridPerResident * resident, a.max_grid);
  hipLaunchKernelGGL((attnres_bwd_block_kernel<G, CH, T, VEC, Rows, Grads>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kBlock), 0, stream, a);
  return blocks;
}

// The (64, 4) token-block backward is compiled in a translation unit of its
// own (ATTNRES_MAX_ILP_UNIT, end of file) with LLVM's max-ilp machine
// scheduler; the (64, 4) geometry unit only declares it.  Measured on MI355X
// (backward alone, us, default scheduler -> max-ilp, two boxes): c2 597.2 /
// 599.4 / 594.7 / 603.1 -> 589.5 / 586.3 / 587.5 / 593.9; S = 13, N = 32768:
// 663.3 -> 656.2; S = 49, N = 8192: 568.4 -> 560.7; S = 24: 576.5 -> 572.5;
// S = 16: 401.5 -> 395.6.  The same scheduler for the whole unit made the
// forward 3-10% slower; for the (64, 8) unit it was within +-0.6%.  LLVM's
// iterative-minreg strategy made this kernel slower (three rounds, us, max-ilp
// -> minreg: c2 583.7-592.0 -> 604.0-613.0; S = 13, N = 32768 646.6-653.4 ->
// 665.2-671.6; S = 49, N = 8192 558.0-562.5 -> 578.1-581.6).  Results are
// bit-identical: only the instruction order changes.
#if defined(ATTNRES_LANES) && defined(ATTNRES_CHUNKS) && ATTNRES_LANES == 64 && ATTNRES_CHUNKS == 4
extern template int64_t launch_bwd_block<64, 4, kBwdBlockTokens, true, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, hipStream_t);
extern template int64_t launch_bwd_block<64, 4, kBwdBlockTokens, true, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, hipStream_t);
#endif

template <int G, int CH, bool NOMASK, bool VEC, bool ACC, class Rows, class Grads>
int64_t launch_bwd(const BwdArgs<Rows, Grads>& a, hipStream_t stream) {
  if constexpr (kBwdBlockVariant<G, CH, NOMASK, VEC, ACC, Grads>) {
    if (a.n_sources >= kBwdBlockMinSources) return launch_bwd_block<G, CH, kBwdBlockTokens, VEC>(a, stream);
  }
  if constexpr (kBwdTwoRowVariant<CH, VEC, ACC> && G >= 64) {
    return launch_bwd_ring<G, CH, 2, NOMASK, VEC, ACC>(a, stream);
  } else if constexpr (kBwdTwoRowVariant<CH, VEC, ACC>) {
    return few_waves(a.n_tokens, G) ? launch_bwd_ring<G, CH, 2, NOMASK, VEC, ACC>(a, stream)
                                    : launch_bwd_ring<G, CH, 1, NOMASK, VEC, ACC>(a, stream);
  } else {
    return launch_bwd_ring<G, CH, 1, NOMASK, VEC, ACC>(a, stream);
  }
}

template <int G, int CH, bool ACC, class Rows, class Grads>
int64_t launch_bwd_variant(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, hipStream_t stream) {
  if (nomask) return vec ? launch_bwd<G, CH, true, true, ACC>(a, stream) : launch_bwd<G, CH, true, false, ACC>(a, stream);
  return vec ? launch_bwd<G, CH, false, true, ACC>(a, stream) : launch_bwd<G, CH, false, false, ACC>(a, stream);
}

template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_geometry(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, bool acc, hipStream_t stream) {
  return acc ? launch_bwd_variant<G, CH, true>(a, nomask, vec, stream)
             : launch_bwd_variant<G, CH, false>(a, nomask, vec, stream);
}

template <int G, int CH, int SM, bool NOMASK, bool VEC, class Rows, class Grads>
int64_t launch_bwd_recompute_rows(const BwdArgs<Rows, Grads>& a, hipStream_t stream) {
  const int64_t resident = resident_blocks<&attnres_bwd_recompute_kernel<G, CH, SM, NOMASK, VEC, Rows, Grads>>();
  const int64_t blocks = grid_blocks(a.n_tokens, G, resident, a.max_grid);
  hipLaunchKernelGGL((attnres_bwd_recompute_kernel<G, CH, SM, NOMASK, VEC, Rows, Grads>),
                     dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream, a);
  return blocks;
}

// Rows held per lane: 3 for reads of at most 3 sources, else the policy's
// maximum.
template <int G, int CH, bool NOMASK, bool VEC, class Rows, class Grads>
int64_t launch_bwd_recompute(const BwdArgs<Rows, Grads>& a, hipStream_t stream) {
  constexpr int kFew = kRecomputeMaxSources < 3 ? kRecomputeMaxSources : 3;
  if (a.n_sources <= kFew) return launch_bwd_recompute_rows<G, CH, kFew, NOMASK, VEC>(a, stream);
  return launch_bwd_recompute_rows<G, CH, kRecomputeMaxSources, NOMASK, VEC>(a, stream);
}

// The key-resident backward for reads of kRecomputeMaxSources < S <=
// kKeyResMaxSources whose key is KC = keyres_key_chunks(D, R) whole chunk
// columns (the host checks this before choosing the recompute path).
// Two rows in flight per group (four were slower or spilled); rows of 4096
// (8 chunks per lane) write each dv row whole, one token later (LAG).
// Measured on MI355X (fwd + bwd per read, us; saved refinement -> key-resident
// with the key part one token later -> whole rows one token later):
// S = 16, N = 16384, D = 4096, R = 1024 (c3): 1207.8 -> 1207.1 -> 1198.7;
// S = 9, D = 4096, R = 1024: 734.7 -> 713.7 -> 713.1; S = 13, D = 4096,
// R = 512: 1011.9 -> 998.3 -> 1000.7; S = 9, N = 32768, D = 2048, R = 1024:
// 723.6 -> 708.1 -> 715.7; S = 16, D = 2048, R = 512: 598.9 -> 594.1 ->
// 591.4.  The forward, which stores no refinement, gains most of it
// (c3: 390 -> 372 us); the backward moves 4% fewer bytes at about the same
// time.  A first version that formed every key part at the token's end (two
// rows in flight over that burst) took 862 us for the c3 backward.
//
// The whole 2048-wide row as key (KC = CH = 4, up to 12 sources, 192 VGPRs of
// held rows; 256 VGPRs + 202 AGPRs aligned) streams the rows the recompute
// kernel holds all at once.  Measured on MI355X (fwd + bwd per read, us, saved
// refinement -> key-resident, D = R = 2048): S = 9, N = 32768 (c4's shape):
// 722.1 -> 698.7; S = 7: 299.7 -> 291.6; S = 12: 459.0 -> 446.7; S = 9,
// N = 16384: 358.6 -> 352.4.
//
// Padding items (S odd, and the items past a group's last token) first
// re-read the group's first row, which the stream had evicted from L2 by then:
// 4.4% extra HBM reads at c4's shape (rocprofv3 FETCH_SIZE).  Measured on
// MI355X (fwd + bwd per read, us; that row -> no load for 4096-wide rows, one
// row shared by all groups for 2048-wide rows): S = 16, D = 4096, R = 1024
// (c3): 1196.0 -> 1166.9 (the backward 825.8 -> 795.3, although c3 pads
// only past a group's last token: the branch changes the compiled schedule);
// S = 15: 1140.8 -> 1100.2; S = 7:
// 578.8 -> 539.0; S = 13, R = 512: 998.0 -> 958.2; S = 9, N = 32768,
// D = R = 2048 (c4's shape): 699.0 -> 680.7; S = 11, D = R = 2048: 419.3 ->
// 411.9; S = 12: 449.7 -> 445.0; S = 11, D = 2048, R = 1024: 433.3 -> 428.6.
// Skipping the load for 2048-wide rows was slower (c4's shape 708.4, S = 12
// 472.3), and the shared row at S = 16, D = 2048, R = 512 too (593.0 ->
// 604.1), so that key keeps the group's first row.
template <int G, int CH, int KC, bool VEC, class Rows, class Grads>
int64_t launch_bwd_keyres_chunks(const BwdArgs<Rows, Grads>& a, hipStream_t stream) {
  constexpr int NB = 2;
  constexpr bool LAG = CH == 8;
  constexpr int KS = keyres_max_sources(KC);
  const int64_t resident = resident_blocks<&attnres_bwd_keyres_kernel<G, CH, KC, KS, NB, LAG, VEC, Rows, Grads>>();
  const int64_t blocks = grid_blocks(a.n_tokens, G, kBwdGridPerResident * resident, a.max_grid);
  hipLaunchKernelGGL((attnres_bwd_keyres_kernel<G, CH, KC, KS, NB, LAG, VEC, Rows, Grads>),
                     dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream, a);
  return blocks;
}

// The whole-row key-resident backward (64 lanes x 4 chunks, D = R = 2048) is
// compiled in the max-ilp unit too.  Measured on MI355X (c4's shape, S = 9,
// N = 32768, fwd + bwd loop, backward us, two rounds, default -> max-ilp):
// 457.3 / 455.4 -> 452.8 / 450.5.
#if defined(ATTNRES_LANES) && defined(ATTNRES_CHUNKS) && ATTNRES_LANES == 64 && ATTNRES_CHUNKS == 4
extern template int64_t launch_bwd_keyres_chunks<64, 4, 4, true, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, hipStream_t);
extern template int64_t launch_bwd_keyres_chunks<64, 4, 4, false, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, hipStream_t);
extern template int64_t launch_bwd_keyres_chunks<64, 4, 4, true, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, hipStream_t);
extern template int64_t launch_bwd_keyres_chunks<64, 4, 4, false, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, hipStream_t);
#endif

template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_keyres(const BwdArgs<Rows, Grads>& a, bool vec, hipStream_t stream) {
  if constexpr (G == 64 && CH > kKeyResMaxChunks) {
    switch (keyres_key_chunks(a.width, a.rank)) {
      case 1: return vec ? launch_bwd_keyres_chunks<G, CH, 1, true>(a, stream)
                         : launch_bwd_keyres_chunks<G, CH, 1, false>(a, stream);
      case 2: return vec ? launch_bwd_keyres_chunks<G, CH, 2, true>(a, stream)
                         : launch_bwd_keyres_chunks<G, CH, 2, false>(a, stream);
      case kKeyResFullChunks:
        if constexpr (CH == kKeyResFullChunks) {
          return vec ? launch_bwd_keyres_chunks<G, CH, CH, true>(a, stream)
                     : launch_bwd_keyres_chunks<G, CH, CH, false>(a, stream);
        }
        break;
      default: break;
    }
  }
  return 0;  // not reached: the host accepts such reads only where keyres_key_chunks applies
}

// The recompute kernel keeps S rows per lane: for the (64, 8) geometry
// (2048 < D <= 4096) it runs with a whole workgroup per token instead, two
// chunks per lane (same lane positions covered, so the same NOMASK rule);
// its grid counts those groups (one token per workgroup).
template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_recompute_geometry(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, hipStream_t stream) {
  if (a.n_sources > kRecomputeMaxSources) return launch_bwd_keyres<G, CH>(a, vec, stream);
  constexpr int RG = recompute_lanes(G, CH);
  constexpr int RCH = G * CH / RG;
  static_assert(RG * RCH == G * CH, "same row coverage");
  if (nomask) {
    return vec ? launch_bwd_recompute<RG, RCH, true, true>(a, stream)
               : launch_bwd_recompute<RG, RCH, true, false>(a, stream);
  }
  return vec ? launch_bwd_recompute<RG, RCH, false, true>(a, stream)
             : launch_bwd_recompute<RG, RCH, false, false>(a, stream);
}

template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_geometry_f32(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, hipStream_t stream) {
  return launch_bwd_variant<G, CH, true>(a, nomask, vec, stream);
}

template <int G, int CH, class Rows>
int64_t launch_bwd_geometry_coef(const BwdArgs<Rows, CoefSink>& a, bool nomask, bool vec, hipStream_t stream) {
  return launch_bwd_variant<G, CH, false>(a, nomask, vec, stream);
}

template <int G, int CH, bool VEC, bool BF16OUT, int RING>
void launch_gather_ring(const GatherArgs& a, hipStream_t stream) {
  // the grid of the row geometry's token groups (the gather's own groups are
  // wider: it has no group sums and spreads a row over up to a workgroup)
  const int64_t blocks = grid_blocks(a.n_tokens, geometry(a.width).lanes,
                                     resident_blocks<&attnres_gather_kernel<G, CH, VEC, BF16OUT, RING>>());
  hipLaunchKernelGGL((attnres_gather_kernel<G, CH, VEC, BF16OUT, RING>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kBlock), 0, stream, a);
}

// Gather ring depth: two reads in flight per group, three on small grids
// (at most 4 wavefronts per CU) with at least 16 reads.  Measured on MI355X
// (N tokens, D = 1024, us, two -> three): N = 2048: 48 reads 38.4 -> 34.9,
// 25 reads 22.7 -> 21.4, 8 reads 11.1 -> 11.7; N = 16384, 25 reads:
// 157.7 -> 165.9.
template <int G, int CH, bool VEC, bool BF16OUT>
void launch_gather(const GatherArgs& a, hipStream_t stream) {
  constexpr int T = CH >= 4 ? 1 : 4 / CH;
  if (a.n_reads >= 16 && few_waves((a.n_tokens + T - 1) / T, G)) {
    launch_gather_ring<G, CH, VEC, BF16OUT, 3>(a, stream);
  } else {
    launch_gather_ring<G, CH, VEC, BF16OUT, 2>(a, stream);
  }
}

// The gather has no group sums, so a row is spread over up to a whole
// workgroup with as few chunks per lane as the width allows (fewer registers:
// 64 lanes x 4 chunks took 204 VGPRs, 256 x 1 far fewer).
template <int G, int CH>
void launch_gather_geometry(const GatherArgs& a, bool vec, hipStream_t stream) {
  constexpr int kLanes = G * CH <= kBlock ? G * CH : kBlock;
  constexpr int kChunks = G * CH / kLanes;
  static_assert(kLanes * kChunks == G * CH, "same row coverage");
  if (vec) {
    if (a.bf16_out) launch_gather<kLanes, kChunks, true, true>(a, stream);
    else launch_gather<kLanes, kChunks, true, false>(a, stream);
  } else {
    if (a.bf16_out) launch_gather<kLanes, kChunks, false, true>(a, stream);
    else launch_gather<kLanes, kChunks, false, false>(a, stream);
  }
}

// Translation units: ATTNRES_MAX_ILP_UNIT holds the (64, 4) kernels built with
// the max-ilp scheduler; every other unit holds one row geometry
// (ATTNRES_LANES, ATTNRES_CHUNKS), whole or, with ATTNRES_UNIT_PART, only its
// forward and gather launchers (1) or only its backward launchers (2; for the
// (64, 8) geometry also its masked forwards, see launch_fwd), so that the two
// parts can be built with different scheduler options.
#if defined(ATTNRES_MAX_ILP_UNIT)
template int64_t launch_bwd_block<64, 4, kBwdBlockTokens, true, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, hipStream_t);
template int64_t launch_bwd_block<64, 4, kBwdBlockTokens, true, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, hipStream_t);
template int64_t launch_bwd_keyres_chunks<64, 4, 4, true, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, hipStream_t);
template int64_t launch_bwd_keyres_chunks<64, 4, 4, false, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, hipStream_t);
template int64_t launch_bwd_keyres_chunks<64, 4, 4, true, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, hipStream_t);
template int64_t launch_bwd_keyres_chunks<64, 4, 4, false, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, hipStream_t);
#elif defined(ATTNRES_LANES) && defined(ATTNRES_CHUNKS)
#if !defined(ATTNRES_UNIT_PART) || ATTNRES_UNIT_PART == 1
template void launch_fwd_geometry<ATTNRES_LANES, ATTNRES_CHUNKS, PackedRows>(const FwdArgs<PackedRows>&, bool,
                                                                             bool, hipStream_t);
template void launch_fwd_geometry<ATTNRES_LANES, ATTNRES_CHUNKS, ListRows>(const FwdArgs<ListRows>&, bool, bool,
                                                                           hipStream_t);
template void launch_gather_geometry<ATTNRES_LANES, ATTNRES_CHUNKS>(const GatherArgs&, bool, hipStream_t);
#endif
#if defined(ATTNRES_UNIT_PART) && ATTNRES_UNIT_PART == 2 && ATTNRES_LANES == 64 && ATTNRES_CHUNKS == 8
template void launch_fwd<64, 8, false, true, PackedRows>(const FwdArgs<PackedRows>&, hipStream_t);
template void launch_fwd<64, 8, false, false, PackedRows>(const FwdArgs<PackedRows>&, hipStream_t);
template void launch_fwd<64, 8, false, true, ListRows>(const FwdArgs<ListRows>&, hipStream_t);
template void launch_fwd<64, 8, false, false, ListRows>(const FwdArgs<ListRows>&, hipStream_t);
#endif
#if !defined(ATTNRES_UNIT_PART) || ATTNRES_UNIT_PART == 2
template int64_t launch_bwd_geometry<ATTNRES_LANES, ATTNRES_CHUNKS, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, bool, bool, bool, hipStream_t);
template int64_t launch_bwd_geometry<ATTNRES_LANES, ATTNRES_CHUNKS, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, bool, bool, bool, hipStream_t);
template int64_t launch_bwd_geometry_f32<ATTNRES_LANES, ATTNRES_CHUNKS, PackedRows, PackedGradsF32>(
    const BwdArgs<PackedRows, PackedGradsF32>&, bool, bool, hipStream_t);
template int64_t launch_bwd_geometry_f32<ATTNRES_LANES, ATTNRES_CHUNKS, ListRows, ListGradsF32>(
    const BwdArgs<ListRows, ListGradsF32>&, bool, bool, hipStream_t);
template int64_t launch_bwd_geometry_coef<ATTNRES_LANES, ATTNRES_CHUNKS, PackedRows>(
    const BwdArgs<PackedRows, CoefSink>&, bool, bool, hipStream_t);
template int64_t launch_bwd_geometry_coef<ATTNRES_LANES, ATTNRES_CHUNKS, ListRows>(const BwdArgs<ListRows, CoefSink>&,
                                                                                   bool, bool, hipStream_t);
template int64_t launch_bwd_recompute_geometry<ATTNRES_LANES, ATTNRES_CHUNKS, PackedRows, PackedGrads>(
    const BwdArgs<PackedRows, PackedGrads>&, bool, bool, hipStream_t);
template int64_t launch_bwd_recompute_geometry<ATTNRES_LANES, ATTNRES_CHUNKS, ListRows, ListGrads>(
    const BwdArgs<ListRows, ListGrads>&, bool, bool, hipStream_t);
#endif
#else
#error "compile attnres_kernels.hip with -DATTNRES_LANES=<G> -DATTNRES_CHUNKS=<CH>, or -DATTNRES_MAX_ILP_UNIT"
#endif

}  // namespace attnres_hip
