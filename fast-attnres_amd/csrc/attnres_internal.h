// attnres_internal.h - types shared by the C ABI (attnres_hip.hip) and the
// kernels (attnres_kernels.hip, compiled once per row geometry).
//
// A token row of width D is owned by a group of `lanes` threads; each lane
// holds `chunks` 16-byte chunks (8 BF16 elements) of the row.  The kernels of
// one geometry are instantiated in their own translation unit, so the
// geometries build in parallel.
#ifndef ATTNRES_INTERNAL_H
#define ATTNRES_INTERNAL_H

#include <hip/hip_runtime.h>

#include <cstdint>

#include "attnres_hip.h"

namespace attnres_hip {

constexpr int kMaxSources = ATTNRES_MAX_SOURCES;
constexpr int kMaxWidth = ATTNRES_MAX_WIDTH;
constexpr int kBlock = 256;           // threads per workgroup (4 wavefronts)
constexpr int kVec = 8;               // BF16 elements per chunk (16 bytes)
constexpr int kMaxGridBlocks = 2048;  // persistent grid cap
// Save/recompute policy: reads of at most this many sources save no output
// refinement; their backward derives delta from the value rows.
constexpr int kRecomputeMaxSources = ATTNRES_RECOMPUTE_MAX_SOURCES;

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

// FP32 gradient sums of packed sources: one contiguous [S, N, D] FP32 buffer
// (the accumulating backward of a source bank writes or adds FP32 dv rows).
struct PackedGradsF32 {
  float* base;
  int64_t source_stride;  // N * D
  __device__ __forceinline__ float* row(int s, int64_t n, int d) const {
    return base + s * source_stride + n * d;
  }
};

// FP32 gradient sums of a source list: one contiguous [N, D] FP32 buffer per
// position (the slots of a source bank read as a list).
struct ListGradsF32 {
  float* ptr[kMaxSources];
  __device__ __forceinline__ float* row(int s, int64_t n, int d) const {
    return ptr[s] + n * d;
  }
};

// The coefficient backward of a source bank writes, instead of dv rows, the
// per-(token, source) terms of dv = p dO + a q + [key] b v as three FP32
// planes [3, S, N] (p, a, b; tokens contiguous); the slots' gradients are
// gathered later from the reads' dO rows.
struct CoefSink {
  float* coef;
};

// Gradient types whose rows are FP32 sums (written or added without rounding).
template <class Grads>
inline constexpr bool kF32Grads = false;
template <>
inline constexpr bool kF32Grads<PackedGradsF32> = true;
template <>
inline constexpr bool kF32Grads<ListGradsF32> = true;

template <class Rows>
struct FwdArgs {
  Rows src;
  const uint16_t* query;  // [R] BF16, contiguous
  uint16_t* out;          // [N, D] BF16, contiguous
  int8_t* out_refine;     // [N, D] low-order correction of out; nullptr: not stored
  float* logit;           // [N, S]
  float* inv_rms;         // [N, S]
  float* stats;           // [2, N]
  int64_t n_tokens;
  int n_sources;
  int width;
  int rank;
  float eps;
  float scale;
};

template <class Rows, class Grads>
struct BwdArgs {
  Rows src;
  Grads grad;
  const uint16_t* query;
  const uint16_t* out;       // [N, D] BF16 forward output, contiguous (unused by the recompute kernel)
  const int8_t* out_refine;  // [N, D] its low-order correction (likewise)
  const uint16_t* grad_out;  // [N, D] BF16, contiguous
  const float* logit;
  const float* inv_rms;
  const float* stats;
  float* partial;            // [gridDim.x, R] FP32 dq partial rows
  int64_t max_grid;          // host side only: the launch may not exceed this many workgroups
                             // (the partial rows `partial` holds); the kernels ignore it
  int64_t n_tokens;
  int n_sources;
  int width;
  int rank;
  float scale;
  // Accumulating backward only: bit s set -> source s's gradient rows hold a
  // gradient that dv is added to (bf16(old + dv)); clear -> dv is written.
  uint64_t accumulate[(kMaxSources + 63) / 64];
  __host__ __device__ bool accumulates(int s) const { return (accumulate[s >> 6] >> (s & 63)) & 1u; }
};

// One read that saw the slot being gathered (see attnres_hip_bank_gather).
constexpr int kMaxGatherReads = ATTNRES_MAX_GATHER_READS;  // per launch; more reads take further,
                                                           // accumulating launches
struct GatherRead {
  const uint16_t* grad_out;  // [N, D] BF16 dO of the read
  const uint16_t* qrow;      // [D] BF16: the query on the read's key coordinates, 0 before them
  const float* p;            // [N] plane of the read's coefficients for this slot (a, b follow
                             // at plane_stride and 2 * plane_stride elements)
  int64_t plane_stride;      // S_r * N
};

// The reads of one launch share their query length R (key coordinates
// tail0 = D - R .. D-1), so their b v terms add up to one scalar per token.
struct GatherArgs {
  const uint16_t* values;  // the slot's [N, D] BF16 rows (row n at values + n * row_stride)
  int64_t row_stride;
  void* grad;              // [N, D] contiguous: FP32, or BF16 when bf16_out
  int64_t n_tokens;
  int width;
  int tail0;
  int n_reads;
  int accumulate;          // 1: add to grad (FP32 only), 0: write it
  int bf16_out;            // 1: store the FP32 sums rounded to BF16 (one launch, no accumulate)
  GatherRead read[kMaxGatherReads];
};

// ------------------------------------------------------------------ geometry

struct Geometry {
  int lanes;   // threads per token group
  int chunks;  // 16-byte chunks per lane
};

// Row geometry: 16/32/64 lanes per token (one or several tokens per
// wavefront, no barriers) up to D = 4096, one workgroup per token beyond.
// From D = 257 to 1024 a token takes 32 lanes with 2 or 4 chunks (two tokens
// per wavefront) rather than 64 lanes with 1 or 2: each item's group sum
// then covers twice the bytes.  Measured on MI355X at N = 16384, fwd + bwd:
// D = 1024, S = 9: 200 -> 190 us, S = 25: 490 -> 458, S = 48: 918 -> 885;
// D = 512, S = 25: 264 -> 255.  At D = 2048, 32 x 8 is no faster than 64 x 4
// (it runs at occupancy 1).
inline Geometry geometry(int64_t D) {
  if (D <= 16 * kVec) return {16, 1};
  if (D <= 32 * kVec) return {32, 1};
  if (D <= 64 * kVec) return {32, 2};
  if (D <= 128 * kVec) return {32, 4};
  if (D <= 256 * kVec) return {64, 4};
  if (D <= 512 * kVec) return {64, 8};
  return {256, 4};
}

// Masks can be skipped when every lane position is an in-range key coordinate.
inline bool no_mask(const Geometry& geo, int64_t width, int64_t rank) {
  return rank == width && width == static_cast<int64_t>(geo.lanes) * geo.chunks * kVec;
}

// Key-resident backward (attnres_bwd_keyres_kernel): reads of more than
// kRecomputeMaxSources sources whose rows are full 64-lane geometry rows
// (D = 64 * CH * 8) and whose key is the last KC whole chunk columns
// (R = KC * 512) save no refinement either: the backward keeps the key chunks
// of a token's rows in registers and takes delta from the value rows.  A key
// of 1 or 2 columns (R = 512 or 1024 < D) is held for up to
// kKeyResMaxSources sources; a full row of 4 columns (D = R = 2048) for up to
// kKeyResFullMaxSources.  Returns KC, or 0 where the kernel does not apply.
constexpr int kKeyResMaxSources = ATTNRES_KEYRES_MAX_SOURCES;
constexpr int kKeyResFullMaxSources = ATTNRES_KEYRES_FULL_MAX_SOURCES;
constexpr int kKeyResMaxChunks = 2;
constexpr int kKeyResFullChunks = 4;
inline int keyres_key_chunks(int64_t D, int64_t R) {
  const Geometry geo = geometry(D);
  const int64_t column = static_cast<int64_t>(geo.lanes) * kVec;  // elements per chunk column
  if (geo.lanes != 64 || D != geo.chunks * column || R % column != 0) return 0;
  const int64_t kc = R / column;
  if (kc == geo.chunks) return kc == kKeyResFullChunks ? static_cast<int>(kc) : 0;  // R = D = 2048 only
  return kc <= kKeyResMaxChunks ? static_cast<int>(kc) : 0;
}

// The most sources the key-resident backward holds for a key of kc columns.
constexpr int keyres_max_sources(int kc) { return kc == kKeyResFullChunks ? kKeyResFullMaxSources : kKeyResMaxSources; }

// Whether a read of S sources, width D and rank R can run its backward
// without the saved output and refinement (the save/recompute policy).
inline bool recomputes(int64_t S, int64_t D, int64_t R) {
  if (S <= kRecomputeMaxSources) return true;
  const int kc = keyres_key_chunks(D, R);
  return kc > 0 && S <= keyres_max_sources(kc);
}

// Lanes per token group of the recompute backward: it keeps S rows per lane,
// so for the (64, 8) geometry (2048 < D <= 4096) it runs a whole workgroup
// per token with 2 chunks per lane; every other geometry keeps its group.
constexpr int recompute_lanes(int lanes, int chunks) { return lanes == 64 && chunks == 8 ? kBlock : lanes; }

// Grid for N tokens in groups of `group_lanes` lanes whose groups stride over
// the tokens: one group per token at most, capped by `resident` (the
// workgroups that stay resident on the device, or a multiple of them; <= 0:
// unknown), by kMaxGridBlocks and by `cap` (<= 0: none; the dq partial rows
// the caller's buffer holds).
inline int64_t grid_blocks(int64_t N, int group_lanes, int64_t resident, int64_t cap = 0) {
  const int64_t groups = kBlock / group_lanes;
  int64_t blocks = (N + groups - 1) / groups;
  if (resident > 0 && blocks > resident) blocks = resident;
  if (cap > 0 && blocks > cap) blocks = cap;
  return blocks < kMaxGridBlocks ? blocks : kMaxGridBlocks;
}

// The most workgroups any backward variant launches for N tokens of width D
// (the streaming kernel with the geometry's groups, the recompute kernel with
// recompute_lanes), i.e. the dq partial rows a workspace must hold.
inline int64_t max_grid_rows(int64_t N, int64_t D) {
  const Geometry geo = geometry(D);
  const int lanes = recompute_lanes(geo.lanes, geo.chunks) > geo.lanes ? recompute_lanes(geo.lanes, geo.chunks)
                                                                        : geo.lanes;
  return grid_blocks(N, lanes, 0);
}

// ----------------------------------------------------------------- launchers
// Defined in attnres_kernels.hip, one explicit instantiation per geometry.

// Enqueue the forward of geometry (G, CH) on `stream`.
template <int G, int CH, class Rows>
void launch_fwd_geometry(const FwdArgs<Rows>& a, bool nomask, bool vec, hipStream_t stream);

// Enqueue the backward of geometry (G, CH); returns the grid size (the number
// of dq partial rows written to a.partial).  `acc`: the accumulating variant
// (dv added to the gradient rows of the sources flagged in a.accumulate).
template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_geometry(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, bool acc, hipStream_t stream);

#define ATTNRES_DECLARE_GEOMETRY(G, CH)                                                                  \
  extern template void launch_fwd_geometry<G, CH, PackedRows>(const FwdArgs<PackedRows>&, bool, bool,    \
                                                              hipStream_t);                              \
  extern template void launch_fwd_geometry<G, CH, ListRows>(const FwdArgs<ListRows>&, bool, bool,        \
                                                            hipStream_t);                                \
  extern template int64_t launch_bwd_geometry<G, CH, PackedRows, PackedGrads>(                           \
      const BwdArgs<PackedRows, PackedGrads>&, bool, bool, bool, hipStream_t);                           \
  extern template int64_t launch_bwd_geometry<G, CH, ListRows, ListGrads>(                               \
      const BwdArgs<ListRows, ListGrads>&, bool, bool, bool, hipStream_t);

// Enqueue the recompute-policy backward (n_sources <= kRecomputeMaxSources;
// reads no saved output or refinement); returns the grid size.
template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_recompute_geometry(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, hipStream_t stream);

#define ATTNRES_DECLARE_GEOMETRY_RECOMPUTE(G, CH)                                               \
  extern template int64_t launch_bwd_recompute_geometry<G, CH, PackedRows, PackedGrads>(        \
      const BwdArgs<PackedRows, PackedGrads>&, bool, bool, hipStream_t);                        \
  extern template int64_t launch_bwd_recompute_geometry<G, CH, ListRows, ListGrads>(            \
      const BwdArgs<ListRows, ListGrads>&, bool, bool, hipStream_t);

// The coefficient backward (dz instead of dv) and the slot gather.
template <int G, int CH, class Rows>
int64_t launch_bwd_geometry_coef(const BwdArgs<Rows, CoefSink>& a, bool nomask, bool vec, hipStream_t stream);
template <int G, int CH>
void launch_gather_geometry(const GatherArgs& a, bool vec, hipStream_t stream);  // bf16_out read from a

#define ATTNRES_DECLARE_GEOMETRY_COEF(G, CH)                                                                 \
  extern template int64_t launch_bwd_geometry_coef<G, CH, PackedRows>(const BwdArgs<PackedRows, CoefSink>&, \
                                                                      bool, bool, hipStream_t);              \
  extern template int64_t launch_bwd_geometry_coef<G, CH, ListRows>(const BwdArgs<ListRows, CoefSink>&,     \
                                                                    bool, bool, hipStream_t);                \
  extern template void launch_gather_geometry<G, CH>(const GatherArgs&, bool, hipStream_t);

// The accumulating backward into FP32 gradient sums.
template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_geometry_f32(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, hipStream_t stream);

#define ATTNRES_DECLARE_GEOMETRY_F32(G, CH)                                                       \
  extern template int64_t launch_bwd_geometry_f32<G, CH, PackedRows, PackedGradsF32>(             \
      const BwdArgs<PackedRows, PackedGradsF32>&, bool, bool, hipStream_t);                       \
  extern template int64_t launch_bwd_geometry_f32<G, CH, ListRows, ListGradsF32>(                 \
      const BwdArgs<ListRows, ListGradsF32>&, bool, bool, hipStream_t);

#define ATTNRES_FOR_EACH_GEOMETRY(X) X(16, 1) X(32, 1) X(32, 2) X(32, 4) X(64, 4) X(64, 8) X(256, 4)

}  // namespace attnres_hip

#endif  // ATTNRES_INTERNAL_H
