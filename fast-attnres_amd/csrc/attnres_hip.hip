// attnres_hip.hip - C ABI of the MI355X (gfx950) Fast-AttnRes read.
//
// Host-side argument checks, dispatch to the kernels of the row geometry
// (attnres_kernels.hip, one translation unit per geometry) and the
// deterministic one-launch reduction of the dq partial rows.  Nothing here
// allocates, synchronises or reads device memory: every entry point only
// enqueues work on the caller's stream.
//
// Reference behaviour followed: the launches inside the ops of
// src/attnres/_kernels/fixed_tail.py:904-1034 (packed) and
// src/attnres/_kernels/fixed_tail_sources.py:78-102 via
// src/attnres/_kernels/fla_full_sources.py:752-942 (source list).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <type_traits>

#include "attnres_internal.h"

// The dq workspace of attnres_hip_packed_backward_noalloc: device memory the
// library holds for the life of the process, one copy per GPU (4 MiB each).
// Its host-side name is not a device address: host code uses the address
// hipGetSymbolAddress returns on each device (attnres_hip::device_scratch).
// Nothing in it needs clearing: every backward workgroup writes its whole
// dq partial row, and the reduction reads only the rows of its own launch.
static constexpr int64_t kScratchElems = int64_t{1} << 20;  // FP32
static __device__ __align__(256) float scratch[kScratchElems];

namespace attnres_hip {

ATTNRES_FOR_EACH_GEOMETRY(ATTNRES_DECLARE_GEOMETRY)
ATTNRES_FOR_EACH_GEOMETRY(ATTNRES_DECLARE_GEOMETRY_F32)
ATTNRES_FOR_EACH_GEOMETRY(ATTNRES_DECLARE_GEOMETRY_RECOMPUTE)
ATTNRES_FOR_EACH_GEOMETRY(ATTNRES_DECLARE_GEOMETRY_COEF)

namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// FP32 to BF16, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t to_bf16(float x) {
  f32x2 v = {x, 0.0f};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return static_cast<uint16_t>(__builtin_bit_cast(uint32_t, b) & 0xffffu);
}

// Two FP32 values to packed BF16 (low element first), round-to-nearest-even.
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// The dq reduction, one launch over the backward's per-block partial rows
// (a few MB, latency-bound).  Workgroup w owns columns [16w, 16w + 16); its
// threads are 16 columns x 16 row groups, and row group g sums rows g, g + 16,
// g + 32, ... in that order, issuing kDqBatch loads at once (clamped,
// unconditional indices; the clamped values are skipped with a select, so the
// sums are exactly the in-order sums).  The 16 group sums meet in LDS and are
// added in group order: a fixed order for a given row count, so dq is
// bit-reproducible.  Writes the FP32 total and its BF16 copy.  The batch size
// does not change the order of the sums.  Measured on MI355X (backward op,
// us, batch 16 -> 8): c2 588.5 -> 582.6; S = 25, N = 16384, D = 1024: 309.9
// -> 303.4; S = 9, N = 32768, D = 2048: 478.9 -> 475.5; S = 25, N = 2048,
// D = 1024: 44.3 -> 42.5 (batches of 4 and 32 in between).
constexpr int kDqCols = 16;
constexpr int kDqGroups = kBlock / kDqCols;
constexpr int kDqBatch = 8;

__global__ void __launch_bounds__(kBlock) attnres_dq_reduce_kernel(
    const float* __restrict__ partial, int64_t rows, int R, float* __restrict__ dq32,
    uint16_t* __restrict__ dq16) {
  __shared__ float sums[kDqGroups][kDqCols];
  const int c = threadIdx.x % kDqCols;
  const int g = threadIdx.x / kDqCols;
  const int col = blockIdx.x * kDqCols + c;
  const int at = col < R ? col : R - 1;
  float t = 0.0f;
  for (int64_t base = g; base < rows; base += static_cast<int64_t>(kDqGroups) * kDqBatch) {
    float v[kDqBatch];
#pragma unroll
    for (int k = 0; k < kDqBatch; ++k) {
      const int64_t r = base + static_cast<int64_t>(k) * kDqGroups;
      v[k] = partial[(r < rows ? r : base) * R + at];
    }
#pragma unroll
    for (int k = 0; k < kDqBatch; ++k) t = base + static_cast<int64_t>(k) * kDqGroups < rows ? t + v[k] : t;
  }
  sums[g][c] = t;
  __syncthreads();
  if (g == 0 && col < R) {
    float total = 0.0f;
#pragma unroll
    for (int k = 0; k < kDqGroups; ++k) total += sums[k][c];
    dq32[col] = total;
    dq16[col] = to_bf16(total);
  }
}

// Block-schedule partial sum: out = prev + emitted in FP32 arithmetic, stored
// in the inputs' dtype (T), and bf16(out) for the read that takes the partial
// as a source -- the add and the BF16 staging in one pass.  Thread i handles
// elements [8i, 8i + 8): 16/32-byte loads and stores when VEC (pointers 16-byte
// aligned and n % 8 == 0), else element by element.
template <typename T>
__device__ __forceinline__ float load_as_f32(const T* p, int64_t i) {
  if constexpr (std::is_same_v<T, float>) {
    return p[i];
  } else {
    return __uint_as_float(static_cast<uint32_t>(p[i]) << 16);
  }
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(kBlock) attnres_partial_sum_kernel(const T* __restrict__ prev,
                                                                     const T* __restrict__ emitted, int64_t n,
                                                                     T* __restrict__ out,
                                                                     uint16_t* __restrict__ out_bf16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * kVec;
  for (int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * kVec; i0 < n; i0 += stride) {
    float x[kVec];
    if constexpr (VEC) {
      if constexpr (std::is_same_v<T, float>) {
        const f32x4* a = reinterpret_cast<const f32x4*>(prev + i0);
        const f32x4* b = reinterpret_cast<const f32x4*>(emitted + i0);
        const f32x4 a0 = __builtin_nontemporal_load(a), a1 = __builtin_nontemporal_load(a + 1);
        const f32x4 b0 = __builtin_nontemporal_load(b), b1 = __builtin_nontemporal_load(b + 1);
        const f32x4 s0 = a0 + b0, s1 = a1 + b1;
        __builtin_nontemporal_store(s0, reinterpret_cast<f32x4*>(out + i0));
        __builtin_nontemporal_store(s1, reinterpret_cast<f32x4*>(out + i0) + 1);
        x[0] = s0.x; x[1] = s0.y; x[2] = s0.z; x[3] = s0.w;
        x[4] = s1.x; x[5] = s1.y; x[6] = s1.z; x[7] = s1.w;
      } else {
        const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(prev + i0));
        const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(emitted + i0));
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[2 * j] = __uint_as_float(aw[j] << 16) + __uint_as_float(bw[j] << 16);
          x[2 * j + 1] = __uint_as_float(aw[j] & 0xffff0000u) + __uint_as_float(bw[j] & 0xffff0000u);
        }
      }
      u32x4 w;
      w.x = pack2_bf16(x[0], x[1]);
      w.y = pack2_bf16(x[2], x[3]);
      w.z = pack2_bf16(x[4], x[5]);
      w.w = pack2_bf16(x[6], x[7]);
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(out_bf16 + i0));
      if constexpr (!std::is_same_v<T, float>) __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(out + i0));
    } else {
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        const int64_t i = i0 + e;
        if (i < n) {
          const float v = load_as_f32(prev, i) + load_as_f32(emitted, i);
          const uint16_t h = to_bf16(v);
          out_bf16[i] = h;
          if constexpr (std::is_same_v<T, float>) {
            out[i] = v;
          } else {
            out[i] = h;
          }
        }
      }
    }
  }
}

int launch_status(const char* what);

int launch_partial_sum(const void* prev, const void* emitted, bool f32, int64_t n, void* out, void* out_bf16,
                       hipStream_t stream) {
  const bool vec = n % kVec == 0 && ((reinterpret_cast<uintptr_t>(prev) | reinterpret_cast<uintptr_t>(emitted) |
                                      reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(out_bf16)) &
                                     15u) == 0;
  const int64_t threads = (n + kVec - 1) / kVec;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((threads + kBlock - 1) / kBlock, 65536));
  if (f32) {
    if (vec) {
      hipLaunchKernelGGL((attnres_partial_sum_kernel<float, true>), dim3(blocks), dim3(kBlock), 0, stream,
                         static_cast<const float*>(prev), static_cast<const float*>(emitted), n,
                         static_cast<float*>(out), static_cast<uint16_t*>(out_bf16));
    } else {
      hipLaunchKernelGGL((attnres_partial_sum_kernel<float, false>), dim3(blocks), dim3(kBlock), 0, stream,
                         static_cast<const float*>(prev), static_cast<const float*>(emitted), n,
                         static_cast<float*>(out), static_cast<uint16_t*>(out_bf16));
    }
  } else {
    if (vec) {
      hipLaunchKernelGGL((attnres_partial_sum_kernel<uint16_t, true>), dim3(blocks), dim3(kBlock), 0, stream,
                         static_cast<const uint16_t*>(prev), static_cast<const uint16_t*>(emitted), n,
                         static_cast<uint16_t*>(out), static_cast<uint16_t*>(out_bf16));
    } else {
      hipLaunchKernelGGL((attnres_partial_sum_kernel<uint16_t, false>), dim3(blocks), dim3(kBlock), 0, stream,
                         static_cast<const uint16_t*>(prev), static_cast<const uint16_t*>(emitted), n,
                         static_cast<uint16_t*>(out), static_cast<uint16_t*>(out_bf16));
    }
  }
  return launch_status("attnres partial sum");
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ATTNRES_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return ATTNRES_OK;
}

template <class Rows>
int launch_forward(const FwdArgs<Rows>& a, bool vec, hipStream_t stream) {
  const Geometry geo = geometry(a.width);
  const bool nomask = no_mask(geo, a.width, a.rank);
  switch (geo.lanes * 100 + geo.chunks) {
    case 1601: launch_fwd_geometry<16, 1>(a, nomask, vec, stream); break;
    case 3201: launch_fwd_geometry<32, 1>(a, nomask, vec, stream); break;
    case 3202: launch_fwd_geometry<32, 2>(a, nomask, vec, stream); break;
    case 3204: launch_fwd_geometry<32, 4>(a, nomask, vec, stream); break;
    case 6404: launch_fwd_geometry<64, 4>(a, nomask, vec, stream); break;
    case 6408: launch_fwd_geometry<64, 8>(a, nomask, vec, stream); break;
    default: launch_fwd_geometry<256, 4>(a, nomask, vec, stream); break;
  }
  return launch_status("attnres forward");
}

// BF16 gradients: the plain or the accumulating kernel; FP32 gradient sums:
// always the accumulating kernel (its first write leaves every bit clear).
template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_geometry_any(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, bool acc, hipStream_t stream) {
  if constexpr (kF32Grads<Grads>) {
    (void)acc;
    return launch_bwd_geometry_f32<G, CH>(a, nomask, vec, stream);
  } else {
    return launch_bwd_geometry<G, CH>(a, nomask, vec, acc, stream);
  }
}

// The recompute kernel (no saved refinement) exists for BF16 gradients only.
template <int G, int CH, class Rows, class Grads>
int64_t launch_bwd_select(const BwdArgs<Rows, Grads>& a, bool nomask, bool vec, bool acc, bool recompute,
                          hipStream_t stream) {
  if constexpr (std::is_same_v<Grads, CoefSink>) {
    (void)acc;
    (void)recompute;
    return launch_bwd_geometry_coef<G, CH>(a, nomask, vec, stream);
  } else {
    if constexpr (!kF32Grads<Grads>) {
      if (recompute) return launch_bwd_recompute_geometry<G, CH>(a, nomask, vec, stream);
    }
    return launch_bwd_geometry_any<G, CH>(a, nomask, vec, acc, stream);
  }
}

template <class Rows, class Grads>
int launch_backward(const BwdArgs<Rows, Grads>& a, bool vec, bool acc, bool recompute, float* dq32, uint16_t* dq16,
                    hipStream_t stream) {
  const Geometry geo = geometry(a.width);
  const bool nomask = no_mask(geo, a.width, a.rank);
  int64_t blocks = 0;
  switch (geo.lanes * 100 + geo.chunks) {
    case 1601: blocks = launch_bwd_select<16, 1>(a, nomask, vec, acc, recompute, stream); break;
    case 3201: blocks = launch_bwd_select<32, 1>(a, nomask, vec, acc, recompute, stream); break;
    case 3202: blocks = launch_bwd_select<32, 2>(a, nomask, vec, acc, recompute, stream); break;
    case 3204: blocks = launch_bwd_select<32, 4>(a, nomask, vec, acc, recompute, stream); break;
    case 6404: blocks = launch_bwd_select<64, 4>(a, nomask, vec, acc, recompute, stream); break;
    case 6408: blocks = launch_bwd_select<64, 8>(a, nomask, vec, acc, recompute, stream); break;
    default: blocks = launch_bwd_select<256, 4>(a, nomask, vec, acc, recompute, stream); break;
  }
  int st = launch_status("attnres backward");
  if (st != ATTNRES_OK) return st;
  const unsigned strips = static_cast<unsigned>((a.rank + kDqCols - 1) / kDqCols);
  hipLaunchKernelGGL(attnres_dq_reduce_kernel, dim3(strips), dim3(kBlock), 0, stream, a.partial, blocks, a.rank,
                     dq32, dq16);
  return launch_status("attnres dq reduction");
}

int check_scalars(float eps, float scale, bool need_eps) {
  if (need_eps && !(std::isfinite(eps) && eps > 0.0f)) return fail(ATTNRES_ERR_SCALAR, "eps must be finite and positive");
  if (!std::isfinite(scale)) return fail(ATTNRES_ERR_SCALAR, "scale must be finite");
  return ATTNRES_OK;
}

// Accumulate bits from one flag byte per source (nullptr: none); returns
// whether any source accumulates.
template <class Rows, class Grads>
bool set_accumulate(BwdArgs<Rows, Grads>& a, const uint8_t* flags, int64_t n_sources) {
  bool any = false;
  for (auto& word : a.accumulate) word = 0;
  if (!flags) return false;
  for (int64_t s = 0; s < n_sources; ++s) {
    if (flags[s]) {
      a.accumulate[s >> 6] |= uint64_t{1} << (s & 63);
      any = true;
    }
  }
  return any;
}

// The pointer is 16-byte aligned or absent.
bool aligned16_or_null(const void* p) { return !p || aligned16(p); }

// Backward without the saved output: the recompute kernel, for small reads only.
int check_recompute(bool recompute, int64_t S, int64_t D, int64_t R, const char* name) {
  if (recompute && !recomputes(S, D, R))
    return fail(ATTNRES_ERR_SHAPE,
                "%s without out_refine needs n_sources <= %d, or <= %d with a key of 512 or 1024 whole "
                "columns of a 2048- or 4096-wide row, or <= %d with width = rank = 2048 (got n_sources=%lld, "
                "width=%lld, rank=%lld)",
                name, kRecomputeMaxSources, kKeyResMaxSources, kKeyResFullMaxSources, (long long)S, (long long)D,
                (long long)R);
  return ATTNRES_OK;
}

// Workspace layout (FP32): [max_grid_rows, R] partial rows, [R] total.
int64_t workspace_elems(int64_t N, int64_t D, int64_t R) { return (max_grid_rows(N, D) + 1) * R; }

}  // namespace
}  // namespace attnres_hip

using namespace attnres_hip;

// ------------------------------------------------------------------- C ABI

extern "C" {

const char* attnres_hip_version(void) { return "2.0.1+mi355x.1"; }

const char* attnres_hip_last_error(void) { return g_error; }

int attnres_hip_saves_refinement(int64_t n_sources) { return n_sources > kRecomputeMaxSources ? 1 : 0; }

int attnres_hip_saves_refinement_for(int64_t n_sources, int64_t width, int64_t rank) {
  return recomputes(n_sources, width, rank) ? 0 : 1;
}

int64_t attnres_hip_dq_workspace_elems(int64_t n_tokens, int64_t width, int64_t rank) {
  if (check_shape(1, n_tokens, width, rank) != ATTNRES_OK) return -1;
  return workspace_elems(n_tokens, width, rank);
}

int attnres_hip_packed_forward(const void* values, int64_t source_stride, int64_t row_stride,
                               int64_t n_sources, int64_t n_tokens, int64_t width,
                               const void* query, int64_t rank, float eps, float scale,
                               void* out, int8_t* out_refine, float* logit, float* inv_rms,
                               float* stats, void* stream) {
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  if (!values || !query || !out || !logit || !inv_rms || !stats)
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
  a.eps = eps;
  a.scale = scale;
  const bool vec = width % kVec == 0 && aligned16(values) && aligned16(out) && aligned16_or_null(out_refine) &&
                   (source_stride % kVec == 0 || n_sources == 1) && (row_stride % kVec == 0 || n_tokens == 1);
  return launch_forward(a, vec, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace attnres_hip {
namespace {

// `fit_grid`: a workspace smaller than workspace_elems() caps the backward's
// grid at the partial rows it holds (at least one) instead of being rejected
// -- the kernels stride over tokens, so any grid gives the same dv, and dq
// differs only in the FP32 order of the per-workgroup sums.
template <class Grads = PackedGrads>
int packed_backward(const void* values, int64_t source_stride, int64_t row_stride, int64_t n_sources,
                    int64_t n_tokens, int64_t width, const void* query, int64_t rank, float scale,
                    const void* out, const int8_t* out_refine, const void* grad_out, const float* logit,
                    const float* inv_rms, const float* stats, void* grad_values, void* grad_query,
                    float* dq_workspace, int64_t dq_workspace_elems, const uint8_t* accumulate, bool need_flags,
                    void* stream, bool fit_grid = false, const char* entry = nullptr) {
  constexpr bool kF32 = kF32Grads<Grads>;
  constexpr bool kCoef = std::is_same_v<Grads, CoefSink>;
  const char* name = entry                ? entry
                     : kCoef              ? "attnres_hip_packed_backward_coef"
                     : kF32               ? "attnres_hip_packed_backward_accumulate_f32"
                     : need_flags         ? "attnres_hip_packed_backward_accumulate"
                                          : "attnres_hip_packed_backward";
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  const bool recompute = !kCoef && !need_flags && !out_refine;
  if (!values || !query || (!recompute && (!out || !out_refine)) || !grad_out || !logit || !inv_rms || !stats ||
      !grad_values || !grad_query || !dq_workspace || (need_flags && !accumulate))
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to %s", name);
  if ((st = check_recompute(recompute, n_sources, width, rank, name))) return st;
  if (source_stride < 0 || row_stride < 0) return fail(ATTNRES_ERR_STRIDE, "negative stride in %s", name);
  if ((st = check_scalars(1.0f, scale, false))) return st;
  const int64_t need = workspace_elems(n_tokens, width, rank);
  if (dq_workspace_elems < (fit_grid ? 2 * rank : need))
    return fail(ATTNRES_ERR_WORKSPACE, "dq workspace has %lld elements, needs %lld",
                (long long)dq_workspace_elems, (long long)(fit_grid ? 2 * rank : need));
  const int64_t rows = std::min(need, dq_workspace_elems) / rank - 1;  // partial rows; the total follows
  BwdArgs<PackedRows, Grads> a{};
  a.src = PackedRows{static_cast<const uint16_t*>(values), source_stride, row_stride};
  if constexpr (kCoef) {
    a.grad = CoefSink{static_cast<float*>(grad_values)};  // the coefficient planes
  } else if constexpr (kF32) {
    a.grad = PackedGradsF32{static_cast<float*>(grad_values), n_tokens * width};
  } else {
    a.grad = PackedGrads{static_cast<uint16_t*>(grad_values), n_tokens * width};
  }
  a.query = static_cast<const uint16_t*>(query);
  a.out = static_cast<const uint16_t*>(out);
  a.out_refine = out_refine;
  a.grad_out = static_cast<const uint16_t*>(grad_out);
  a.logit = logit;
  a.inv_rms = inv_rms;
  a.stats = stats;
  a.partial = dq_workspace;
  a.max_grid = rows;
  a.n_tokens = n_tokens;
  a.n_sources = static_cast<int>(n_sources);
  a.width = static_cast<int>(width);
  a.rank = static_cast<int>(rank);
  a.scale = scale;
  const bool vec = width % kVec == 0 && aligned16(values) && aligned16_or_null(out) &&
                   aligned16_or_null(out_refine) && aligned16(grad_out) && (kCoef || aligned16(grad_values)) &&
                   (source_stride % kVec == 0 || n_sources == 1) && (row_stride % kVec == 0 || n_tokens == 1);
  const bool acc = set_accumulate(a, accumulate, n_sources);
  float* dq32 = dq_workspace + rows * rank;  // after the partial rows
  return launch_backward(a, vec, acc, recompute, dq32, static_cast<uint16_t*>(grad_query),
                         static_cast<hipStream_t>(stream));
}

// ------------------------------------------------- scratch of the no-alloc entry

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up on its first use there
// (with that device current, as the caller's stream requires).
int device_scratch(float** ptr) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ATTNRES_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  }
  if (device < 0 || device >= kMaxDevices)
    return fail(ATTNRES_ERR_LAUNCH, "device %d outside 0..%d", device, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void* address = nullptr;
    e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !address) {
      (void)hipGetLastError();
      return fail(ATTNRES_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d failed: %s", device,
                  hipGetErrorString(e));
    }
    g_scratch[device] = static_cast<float*>(address);
  }
  *ptr = g_scratch[device];
  return ATTNRES_OK;
}

}  // namespace
}  // namespace attnres_hip

extern "C" {

int attnres_hip_packed_backward_noalloc(const void* values, int64_t source_stride, int64_t row_stride,
                                        int64_t n_sources, int64_t n_tokens, int64_t width,
                                        const void* query, int64_t rank, float scale, const void* out,
                                        const int8_t* out_refine, const void* grad_out,
                                        const float* logit, const float* inv_rms, const float* stats,
                                        void* grad_values, void* grad_query, void* stream) {
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  if (2 * rank > kScratchElems)
    return fail(ATTNRES_ERR_WORKSPACE, "rank=%lld needs more than the %lld-element scratch", (long long)rank,
                (long long)kScratchElems);
  // every argument check of the workspace entry point, before any runtime call
  static const char* const kName = "attnres_hip_packed_backward_noalloc";
  if (!values || !query || (out_refine && !out) || !grad_out || !logit || !inv_rms || !stats || !grad_values ||
      !grad_query)
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to %s", kName);
  if ((st = check_recompute(!out_refine, n_sources, width, rank, kName))) return st;
  if (source_stride < 0 || row_stride < 0) return fail(ATTNRES_ERR_STRIDE, "negative stride in %s", kName);
  if ((st = check_scalars(1.0f, scale, false))) return st;
  float* workspace = nullptr;
  if ((st = device_scratch(&workspace))) return st;
  return packed_backward(values, source_stride, row_stride, n_sources, n_tokens, width, query, rank, scale, out,
                         out_refine, grad_out, logit, inv_rms, stats, grad_values, grad_query, workspace,
                         kScratchElems, nullptr, false, stream, true, kName);
}

int attnres_hip_packed_backward(const void* values, int64_t source_stride, int64_t row_stride,
                                int64_t n_sources, int64_t n_tokens, int64_t width,
                                const void* query, int64_t rank, float scale, const void* out,
                                const int8_t* out_refine, const void* grad_out,
                                const float* logit, const float* inv_rms, const float* stats,
                                void* grad_values, void* grad_query, float* dq_workspace,
                                int64_t dq_workspace_elems, void* stream) {
  return packed_backward(values, source_stride, row_stride, n_sources, n_tokens, width, query, rank, scale, out,
                         out_refine, grad_out, logit, inv_rms, stats, grad_values, grad_query, dq_workspace,
                         dq_workspace_elems, nullptr, false, stream);
}

int attnres_hip_packed_backward_accumulate(const void* values, int64_t source_stride, int64_t row_stride,
                                           int64_t n_sources, int64_t n_tokens, int64_t width,
                                           const void* query, int64_t rank, float scale, const void* out,
                                           const int8_t* out_refine, const void* grad_out,
                                           const float* logit, const float* inv_rms, const float* stats,
                                           void* grad_values, void* grad_query, float* dq_workspace,
                                           int64_t dq_workspace_elems, const uint8_t* accumulate,
                                           void* stream) {
  return packed_backward(values, source_stride, row_stride, n_sources, n_tokens, width, query, rank, scale, out,
                         out_refine, grad_out, logit, inv_rms, stats, grad_values, grad_query, dq_workspace,
                         dq_workspace_elems, accumulate, true, stream);
}

int attnres_hip_packed_backward_accumulate_f32(const void* values, int64_t source_stride, int64_t row_stride,
                                               int64_t n_sources, int64_t n_tokens, int64_t width,
                                               const void* query, int64_t rank, float scale, const void* out,
                                               const int8_t* out_refine, const void* grad_out,
                                               const float* logit, const float* inv_rms, const float* stats,
                                               float* grad_sums, void* grad_query, float* dq_workspace,
                                               int64_t dq_workspace_elems, const uint8_t* accumulate,
                                               void* stream) {
  return packed_backward<PackedGradsF32>(values, source_stride, row_stride, n_sources, n_tokens, width, query, rank,
                                         scale, out, out_refine, grad_out, logit, inv_rms, stats, grad_sums,
                                         grad_query, dq_workspace, dq_workspace_elems, accumulate, true, stream);
}

int attnres_hip_sources_forward(const void* const* sources, const int64_t* row_strides,
                                int64_t n_sources, int64_t n_tokens, int64_t width,
                                const void* query, int64_t rank, float eps, float scale, void* out,
                                int8_t* out_refine, float* logit, float* inv_rms, float* stats,
                                void* stream) {
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  if (!sources || !row_strides || !query || !out || !logit || !inv_rms || !stats)
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to attnres_hip_sources_forward");
  if ((st = check_scalars(eps, scale, true))) return st;
  FwdArgs<ListRows> a{};
  bool vec = width % kVec == 0 && aligned16(out) && aligned16_or_null(out_refine);
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
  a.eps = eps;
  a.scale = scale;
  return launch_forward(a, vec, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace attnres_hip {
namespace {

template <class Grads = ListGrads>
int sources_backward(const void* const* sources, const int64_t* row_strides, int64_t n_sources,
                     int64_t n_tokens, int64_t width, const void* query, int64_t rank, float scale,
                     const void* out, const int8_t* out_refine, const void* grad_out, const float* logit,
                     const float* inv_rms, const float* stats, void* const* grad_sources, void* grad_query,
                     float* dq_workspace, int64_t dq_workspace_elems, const uint8_t* accumulate, bool need_flags,
                     void* stream, float* coef = nullptr) {
  constexpr bool kF32 = kF32Grads<Grads>;
  constexpr bool kCoef = std::is_same_v<Grads, CoefSink>;
  const char* name = kCoef ? "attnres_hip_sources_backward_coef"
                     : kF32 ? "attnres_hip_sources_backward_accumulate_f32"
                     : need_flags ? "attnres_hip_sources_backward_accumulate" : "attnres_hip_sources_backward";
  int st = check_shape(n_sources, n_tokens, width, rank);
  if (st) return st;
  const bool recompute = !kCoef && !need_flags && !out_refine;
  if (!sources || !row_strides || !query || (!recompute && (!out || !out_refine)) || !grad_out || !logit ||
      !inv_rms || !stats || (kCoef ? !coef : !grad_sources) || !grad_query || !dq_workspace ||
      (need_flags && !accumulate))
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to %s", name);
  if ((st = check_recompute(recompute, n_sources, width, rank, name))) return st;
  if ((st = check_scalars(1.0f, scale, false))) return st;
  const int64_t need = workspace_elems(n_tokens, width, rank);
  if (dq_workspace_elems < need)
    return fail(ATTNRES_ERR_WORKSPACE, "dq workspace has %lld elements, needs %lld",
                (long long)dq_workspace_elems, (long long)need);
  BwdArgs<ListRows, Grads> a{};
  bool vec = width % kVec == 0 && aligned16_or_null(out) && aligned16_or_null(out_refine) && aligned16(grad_out);
  for (int64_t s = 0; s < n_sources; ++s) {
    if (!sources[s] || (!kCoef && !grad_sources[s]))
      return fail(ATTNRES_ERR_NULL_POINTER, "source %lld or its gradient is null", (long long)s);
    if (row_strides[s] < 0) return fail(ATTNRES_ERR_STRIDE, "source %lld has a negative row stride", (long long)s);
    a.src.ptr[s] = static_cast<const uint16_t*>(sources[s]);
    a.src.row_stride[s] = row_strides[s];
    vec = vec && aligned16(sources[s]) && (row_strides[s] % kVec == 0 || n_tokens == 1);
    if constexpr (!kCoef) {
      a.grad.ptr[s] = static_cast<std::remove_reference_t<decltype(a.grad.ptr[0])>>(grad_sources[s]);
      vec = vec && aligned16(grad_sources[s]);
    }
  }
  if constexpr (kCoef) a.grad.coef = coef;
  a.query = static_cast<const uint16_t*>(query);
  a.out = static_cast<const uint16_t*>(out);
  a.out_refine = out_refine;
  a.grad_out = static_cast<const uint16_t*>(grad_out);
  a.logit = logit;
  a.inv_rms = inv_rms;
  a.stats = stats;
  a.partial = dq_workspace;
  a.max_grid = need / rank - 1;
  a.n_tokens = n_tokens;
  a.n_sources = static_cast<int>(n_sources);
  a.width = static_cast<int>(width);
  a.rank = static_cast<int>(rank);
  a.scale = scale;
  const bool acc = set_accumulate(a, accumulate, n_sources);
  float* dq32 = dq_workspace + (need - rank);  // after the partial rows
  return launch_backward(a, vec, acc, recompute, dq32, static_cast<uint16_t*>(grad_query),
                         static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace attnres_hip

extern "C" {

int attnres_hip_sources_backward(const void* const* sources, const int64_t* row_strides,
                                 int64_t n_sources, int64_t n_tokens, int64_t width,
                                 const void* query, int64_t rank, float scale, const void* out,
                                 const int8_t* out_refine, const void* grad_out,
                                 const float* logit, const float* inv_rms, const float* stats,
                                 void* const* grad_sources, void* grad_query, float* dq_workspace,
                                 int64_t dq_workspace_elems, void* stream) {
  return sources_backward(sources, row_strides, n_sources, n_tokens, width, query, rank, scale, out, out_refine,
                          grad_out, logit, inv_rms, stats, grad_sources, grad_query, dq_workspace,
                          dq_workspace_elems, nullptr, false, stream);
}

int attnres_hip_sources_backward_accumulate(const void* const* sources, const int64_t* row_strides,
                                            int64_t n_sources, int64_t n_tokens, int64_t width,
                                            const void* query, int64_t rank, float scale, const void* out,
                                            const int8_t* out_refine, const void* grad_out,
                                            const float* logit, const float* inv_rms, const float* stats,
                                            void* const* grad_sources, void* grad_query, float* dq_workspace,
                                            int64_t dq_workspace_elems, const uint8_t* accumulate,
                                            void* stream) {
  return sources_backward(sources, row_strides, n_sources, n_tokens, width, query, rank, scale, out, out_refine,
                          grad_out, logit, inv_rms, stats, grad_sources, grad_query, dq_workspace,
                          dq_workspace_elems, accumulate, true, stream);
}

int attnres_hip_sources_backward_accumulate_f32(const void* const* sources, const int64_t* row_strides,
                                                int64_t n_sources, int64_t n_tokens, int64_t width,
                                                const void* query, int64_t rank, float scale, const void* out,
                                                const int8_t* out_refine, const void* grad_out,
                                                const float* logit, const float* inv_rms, const float* stats,
                                                float* const* grad_sums, void* grad_query, float* dq_workspace,
                                                int64_t dq_workspace_elems, const uint8_t* accumulate,
                                                void* stream) {
  return sources_backward<ListGradsF32>(sources, row_strides, n_sources, n_tokens, width, query, rank, scale, out,
                                        out_refine, grad_out, logit, inv_rms, stats,
                                        reinterpret_cast<void* const*>(grad_sums), grad_query, dq_workspace,
                                        dq_workspace_elems, accumulate, true, stream);
}

int attnres_hip_packed_backward_coef(const void* values, int64_t source_stride, int64_t row_stride,
                                     int64_t n_sources, int64_t n_tokens, int64_t width, const void* query,
                                     int64_t rank, float scale, const void* out, const int8_t* out_refine,
                                     const void* grad_out, const float* logit, const float* inv_rms,
                                     const float* stats, float* coef, void* grad_query, float* dq_workspace,
                                     int64_t dq_workspace_elems, void* stream) {
  return packed_backward<CoefSink>(values, source_stride, row_stride, n_sources, n_tokens, width, query, rank, scale,
                                   out, out_refine, grad_out, logit, inv_rms, stats, coef, grad_query, dq_workspace,
                                   dq_workspace_elems, nullptr, false, stream);
}

int attnres_hip_sources_backward_coef(const void* const* sources, const int64_t* row_strides, int64_t n_sources,
                                      int64_t n_tokens, int64_t width, const void* query, int64_t rank, float scale,
                                      const void* out, const int8_t* out_refine, const void* grad_out,
                                      const float* logit, const float* inv_rms, const float* stats, float* coef,
                                      void* grad_query, float* dq_workspace, int64_t dq_workspace_elems,
                                      void* stream) {
  return sources_backward<CoefSink>(sources, row_strides, n_sources, n_tokens, width, query, rank, scale, out,
                                    out_refine, grad_out, logit, inv_rms, stats, nullptr, grad_query, dq_workspace,
                                    dq_workspace_elems, nullptr, false, stream, coef);
}

int attnres_hip_bank_gather(const void* values, int64_t row_stride, int64_t n_tokens, int64_t width,
                            const attnres_gather_read* reads, int64_t n_reads, void* grad, int grad_dtype,
                            int accumulate, void* stream) {
  int st = check_shape(1, n_tokens, width, 1);
  if (st) return st;
  if (!values || !reads || !grad) return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to attnres_hip_bank_gather");
  if (row_stride < 0) return fail(ATTNRES_ERR_STRIDE, "negative row stride");
  if (n_reads < 1) return fail(ATTNRES_ERR_SHAPE, "n_reads=%lld must be positive", (long long)n_reads);
  if (grad_dtype != ATTNRES_DTYPE_F32 && grad_dtype != ATTNRES_DTYPE_BF16)
    return fail(ATTNRES_ERR_SHAPE, "grad_dtype=%d is neither ATTNRES_DTYPE_F32 nor ATTNRES_DTYPE_BF16", grad_dtype);
  const bool bf16_out = grad_dtype == ATTNRES_DTYPE_BF16;
  if (bf16_out) {  // one launch, so that the sum is rounded once
    bool one_rank = true;
    for (int64_t r = 1; r < n_reads; ++r) one_rank = one_rank && reads[r].rank == reads[0].rank;
    if (accumulate || n_reads > ATTNRES_MAX_GATHER_READS || !one_rank)
      return fail(ATTNRES_ERR_SHAPE,
                  "a BF16 gradient is written by one launch: accumulate=0, at most %d reads, all of one rank",
                  ATTNRES_MAX_GATHER_READS);
  }
  bool vec = width % kVec == 0 && aligned16(values) && aligned16(grad) && (row_stride % kVec == 0 || n_tokens == 1);
  for (int64_t r = 0; r < n_reads; ++r) {
    const attnres_gather_read& rd = reads[r];
    if (!rd.grad_out || !rd.query_row || !rd.coef)
      return fail(ATTNRES_ERR_NULL_POINTER, "read %lld of attnres_hip_bank_gather has a null pointer", (long long)r);
    if ((st = check_shape(rd.n_sources, n_tokens, width, rd.rank))) return st;
    if (rd.position < 0 || rd.position >= rd.n_sources)
      return fail(ATTNRES_ERR_SHAPE, "read %lld: position %lld outside 0..%lld", (long long)r,
                  (long long)rd.position, (long long)rd.n_sources - 1);
    vec = vec && aligned16(rd.grad_out) && aligned16(rd.query_row);
  }
  // One launch per run of at most kMaxGatherReads reads with the same rank
  // (in the caller's order); every launch after the first adds to grad.
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const Geometry geo = geometry(width);
  bool first_launch = true;
  for (int64_t first = 0; first < n_reads;) {
    GatherArgs a{};
    a.values = static_cast<const uint16_t*>(values);
    a.row_stride = row_stride;
    a.grad = grad;
    a.n_tokens = n_tokens;
    a.width = static_cast<int>(width);
    a.tail0 = static_cast<int>(width - reads[first].rank);
    a.accumulate = (accumulate || !first_launch) ? 1 : 0;
    a.bf16_out = bf16_out ? 1 : 0;
    int count = 0;
    while (first + count < n_reads && count < kMaxGatherReads && reads[first + count].rank == reads[first].rank) {
      const attnres_gather_read& rd = reads[first + count];
      a.read[count++] = GatherRead{static_cast<const uint16_t*>(rd.grad_out),
                                   static_cast<const uint16_t*>(rd.query_row), rd.coef + rd.position * n_tokens,
                                   rd.n_sources * n_tokens};
    }
    a.n_reads = count;
    switch (geo.lanes * 100 + geo.chunks) {
      case 1601: launch_gather_geometry<16, 1>(a, vec, s); break;
      case 3201: launch_gather_geometry<32, 1>(a, vec, s); break;
      case 3202: launch_gather_geometry<32, 2>(a, vec, s); break;
      case 3204: launch_gather_geometry<32, 4>(a, vec, s); break;
      case 6404: launch_gather_geometry<64, 4>(a, vec, s); break;
      case 6408: launch_gather_geometry<64, 8>(a, vec, s); break;
      default: launch_gather_geometry<256, 4>(a, vec, s); break;
    }
    if ((st = launch_status("attnres bank gather")) != ATTNRES_OK) return st;
    first += count;
    first_launch = false;
  }
  return ATTNRES_OK;
}

int attnres_hip_partial_sum(const void* prev, const void* emitted, int dtype, int64_t n_elems, void* out,
                            void* out_bf16, void* stream) {
  if (!prev || !emitted || !out || !out_bf16)
    return fail(ATTNRES_ERR_NULL_POINTER, "null pointer argument to attnres_hip_partial_sum");
  if (dtype != ATTNRES_DTYPE_F32 && dtype != ATTNRES_DTYPE_BF16)
    return fail(ATTNRES_ERR_SHAPE, "dtype=%d is neither ATTNRES_DTYPE_F32 nor ATTNRES_DTYPE_BF16", dtype);
  if (n_elems < 1) return fail(ATTNRES_ERR_SHAPE, "n_elems=%lld must be positive", (long long)n_elems);
  return launch_partial_sum(prev, emitted, dtype == ATTNRES_DTYPE_F32, n_elems, out, out_bf16,
                            static_cast<hipStream_t>(stream));
}

}  // extern "C"
