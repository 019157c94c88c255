// The eager read's autograd nodes, in C++ over the C ABI (attnres_hip.h).
//
// `attnres(values, query)` in eager mode (no dynamo tracing, plain tensors)
// calls `packed_read` / `sources_read` below instead of the torch.library
// ops, which remain the path under torch.compile.  Both launch the same
// kernels on the same saved state, so out, dv and dq are bit-identical
// between them.  What this file saves is host time: the node's forward and
// backward run without Python, and the backward -- which autograd runs on its
// device thread -- takes no Python lock.  On an MI355X box a small read
// (S = 8, N = 1024, D = 1024) costs 80 us of host time for forward plus
// torch.autograd.grad through these nodes, against 139 us through a Python
// autograd.Function, with torch's own floor for a trivial graph at 62 us.
// The packed node also flattens the batch axes itself (two view nodes less
// in the graph): c1's [8, 2, 512, 1024] read 37 us on a box whose floor is
// 29.5 us.  A read that needs no gradient skips the nodes (below).
//
// Saved state: the refinement bytes (when the read saves them) and the FP32
// statistics live in one byte allocation whose addresses are passed to the
// library (layout below), plus the inputs and, for a read that saves its
// refinement, the output.  Reference: the op pair it stands for,
// `attnres::_fixed_tail_forward_with_aux` / `_fixed_tail_backward`
// (fixed_tail.py:904-1034) and the source-list pair (fixed_tail_sources.py:
// 78-183); their autograd registration (fixed_tail.py:1041-1057): the aux
// outputs carry no gradient and a None upstream gradient gives None.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <optional>
#include <vector>

#include "attnres_hip.h"

namespace {

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// A failing status raises as the Python binding does: ValueError for argument
// errors, RuntimeError otherwise, with the library's own message.
void check(int status, const char* what) {
  if (status == ATTNRES_OK) return;
  const char* message = attnres_hip_last_error();
  if (status == ATTNRES_ERR_SHAPE || status == ATTNRES_ERR_STRIDE || status == ATTNRES_ERR_SCALAR ||
      status == ATTNRES_ERR_WORKSPACE) {
    TORCH_CHECK_VALUE(false, what, ": ", message);
  }
  TORCH_CHECK(false, what, ": ", message, " (status ", status, ")");
}

// Pooled saved state: out_refine [N, D] int8 at byte 0 (when saved), then
// from the 16-byte aligned offset `head` logit [N, S], 1/rms [N, S] (`block`
// floats each) and stats [2, N], FP32; `size` bytes in all.  The Python
// `_pool_layout` states the same layout for the ops' pooled views.
struct PoolLayout {
  int64_t head, block, size;
};

PoolLayout pool_layout(int64_t tokens, int64_t sources, int64_t width, bool save) {
  const int64_t head = ((save ? tokens * width : 0) + 15) / 16 * 16;
  const int64_t block = tokens * sources;
  return {head, block, head + 4 * (2 * block + 2 * tokens)};
}

struct StatePointers {
  int8_t* refine;  // nullptr when the read saves no refinement
  float* logit;
  float* inv_rms;
  float* stats;
};

StatePointers pool_pointers(const Tensor& pool, const PoolLayout& layout, bool save) {
  char* base = static_cast<char*>(pool.data_ptr());
  float* logit = reinterpret_cast<float*>(base + layout.head);
  return {save ? reinterpret_cast<int8_t*>(base) : nullptr, logit, logit + layout.block, logit + 2 * layout.block};
}

hipStream_t current_stream(const Tensor& tensor) {
  return c10::hip::getCurrentHIPStream(tensor.device().index()).stream();
}

Tensor bf16_empty(at::IntArrayRef shape, const Tensor& like) {
  return torch::empty(shape, like.options().dtype(torch::kBFloat16));
}

Tensor dq_workspace(int64_t tokens, int64_t width, int64_t rank, const Tensor& like) {
  const int64_t elems = attnres_hip_dq_workspace_elems(tokens, width, rank);
  TORCH_CHECK_VALUE(elems >= 0, "attnres backward: shape outside the supported envelope");
  return torch::empty({elems}, like.options().dtype(torch::kFloat32));
}

// Element stride between consecutive rows of tensor[..., D] flattened to
// [rows, D], or nothing when the rows are not evenly spaced or a row is not
// unit-stride (the Python `row_stride`, after fla_full_sources.py:164-178).
std::optional<int64_t> row_stride(const Tensor& tensor) {
  const int64_t last = tensor.dim() - 1;
  if (tensor.size(last) > 1 && tensor.stride(last) != 1) return std::nullopt;
  std::optional<int64_t> stride;
  int64_t rows = 1;
  for (int64_t d = last - 1; d >= 0; --d) {
    if (tensor.size(d) == 1) continue;
    if (!stride) {
      stride = tensor.stride(d);
    } else if (tensor.stride(d) != rows * *stride) {
      return std::nullopt;
    }
    rows *= tensor.size(d);
  }
  return stride.value_or(0);
}

// Row pointers and strides of a source list; sources whose rows are not
// addressable are copied (the copies live until the launch is enqueued).
struct SourceTable {
  std::vector<Tensor> keep;
  std::vector<const void*> rows;
  std::vector<int64_t> strides;
};

SourceTable source_table(at::TensorList sources) {
  SourceTable table;
  table.keep.reserve(sources.size());
  for (const Tensor& source : sources) {
    Tensor rows = source;
    std::optional<int64_t> stride = row_stride(rows);
    if (!stride) {
      rows = rows.contiguous();
      stride = row_stride(rows);
    }
    table.keep.push_back(rows);
    table.rows.push_back(rows.data_ptr());
    table.strides.push_back(*stride);
  }
  return table;
}

int64_t rows_of(const Tensor& tensor) { return tensor.dim() > 1 ? tensor.numel() / tensor.size(-1) : 1; }

// Packed values [S, ..., D] as rows [S, N, D]: a view where the batch axes
// collapse to one row stride (as torch's reshape does), a copy otherwise, and
// a copy too when a row is not unit-stride.  Called inside a node's forward
// (or with no node at all), so autograd records no view nodes for it.
Tensor flat_rows(const Tensor& values) {
  const int64_t S = values.size(0), D = values.size(-1);
  Tensor rows = values.dim() == 3 ? values : values.reshape({S, -1, D});
  if (D > 1 && rows.stride(2) != 1) rows = rows.contiguous();
  return rows;
}

// ------------------------------------------------------------------ packed

struct PackedRead : public torch::autograd::Function<PackedRead> {
  // values [S, ..., D] (checked by the Python caller), query [R] contiguous.
  // The batch axes flatten to N rows here (flat_rows), so autograd records no
  // view nodes around the read: the output has the batch shape [..., D] and
  // the value gradient the shape of values.
  static Tensor forward(AutogradContext* ctx, const Tensor& values, const Tensor& query, double eps, double scale) {
    const int64_t S = values.size(0), D = values.size(-1), R = query.numel();
    const Tensor rows = flat_rows(values);
    const int64_t N = rows.size(1);
    const bool save = attnres_hip_saves_refinement_for(S, D, R) != 0;
    const c10::DeviceGuard guard(values.device());
    Tensor out = bf16_empty(values.sizes().slice(1), values);  // N contiguous rows
    const PoolLayout layout = pool_layout(N, S, D, save);
    Tensor pool = torch::empty({layout.size}, values.options().dtype(torch::kUInt8));
    const StatePointers state = pool_pointers(pool, layout, save);
    check(attnres_hip_packed_forward(rows.data_ptr(), rows.stride(0), rows.stride(1), S, N, D, query.data_ptr(), R,
                                     static_cast<float>(eps), static_cast<float>(scale), out.data_ptr(), state.refine,
                                     state.logit, state.inv_rms, state.stats, current_stream(values)),
          "attnres packed forward");
    ctx->set_materialize_grads(false);
    if (save) {
      ctx->save_for_backward({rows, query, pool, out});
    } else {
      ctx->save_for_backward({rows, query, pool});
    }
    ctx->saved_data["save"] = save;
    ctx->saved_data["scale"] = scale;
    return out;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    if (!grads[0].defined()) return {Tensor(), Tensor(), Tensor(), Tensor()};
    const variable_list saved = ctx->get_saved_variables();
    const Tensor& rows = saved[0];  // [S, N, D]
    const Tensor& query = saved[1];
    const bool save = ctx->saved_data["save"].toBool();
    const int64_t S = rows.size(0), N = rows.size(1), D = rows.size(2), R = query.numel();
    const c10::DeviceGuard guard(rows.device());
    const Tensor grad_out = grads[0].to(torch::kBFloat16).contiguous();  // the output's shape [..., D]: N rows
    const Tensor out = save ? saved[3].contiguous() : Tensor();
    const StatePointers state = pool_pointers(saved[2], pool_layout(N, S, D, save), save);
    std::vector<int64_t> shape{S};  // the shape of values: [S] + the output's
    shape.insert(shape.end(), grad_out.sizes().begin(), grad_out.sizes().end());
    Tensor grad_values = bf16_empty(shape, rows);
    Tensor grad_query = bf16_empty({R}, rows);
    Tensor workspace = dq_workspace(N, D, R, rows);
    check(attnres_hip_packed_backward(rows.data_ptr(), rows.stride(0), rows.stride(1), S, N, D, query.data_ptr(), R,
                                      static_cast<float>(ctx->saved_data["scale"].toDouble()),
                                      save ? out.data_ptr() : nullptr, state.refine, grad_out.data_ptr(), state.logit,
                                      state.inv_rms, state.stats, grad_values.data_ptr(), grad_query.data_ptr(),
                                      workspace.data_ptr<float>(), workspace.numel(), current_stream(rows)),
          "attnres packed backward");
    return {ctx->needs_input_grad(0) ? grad_values : Tensor(), ctx->needs_input_grad(1) ? grad_query : Tensor(),
            Tensor(), Tensor()};
  }
};

// -------------------------------------------------------------------- list

struct SourcesRead : public torch::autograd::Function<SourcesRead> {
  // sources: S tensors [..., D] of one shape (checked by the Python caller);
  // each list position gets its own gradient.
  static Tensor forward(AutogradContext* ctx, const Tensor& query, double eps, double scale, at::TensorList sources) {
    const Tensor& first = sources[0];
    const int64_t S = static_cast<int64_t>(sources.size()), N = rows_of(first), D = first.size(-1);
    const int64_t R = query.numel();
    const bool save = attnres_hip_saves_refinement_for(S, D, R) != 0;
    const c10::DeviceGuard guard(first.device());
    const SourceTable table = source_table(sources);
    Tensor out = bf16_empty(first.sizes(), first);
    const PoolLayout layout = pool_layout(N, S, D, save);
    Tensor pool = torch::empty({layout.size}, first.options().dtype(torch::kUInt8));
    const StatePointers state = pool_pointers(pool, layout, save);
    check(attnres_hip_sources_forward(table.rows.data(), table.strides.data(), S, N, D, query.data_ptr(), R,
                                      static_cast<float>(eps), static_cast<float>(scale), out.data_ptr(), state.refine,
                                      state.logit, state.inv_rms, state.stats, current_stream(first)),
          "attnres source-list forward");
    ctx->set_materialize_grads(false);
    variable_list keep(sources.begin(), sources.end());
    keep.push_back(query);
    keep.push_back(pool);
    if (save) keep.push_back(out);
    ctx->save_for_backward(keep);
    ctx->saved_data["save"] = save;
    ctx->saved_data["scale"] = scale;
    ctx->saved_data["count"] = S;
    return out;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const int64_t S = ctx->saved_data["count"].toInt();
    variable_list result(3 + S);  // query, eps, scale, then one per source
    if (!grads[0].defined()) return result;
    const variable_list saved = ctx->get_saved_variables();
    const std::vector<Tensor> sources(saved.begin(), saved.begin() + S);
    const Tensor& query = saved[S];
    const bool save = ctx->saved_data["save"].toBool();
    const Tensor& first = sources[0];
    const int64_t N = rows_of(first), D = first.size(-1), R = query.numel();
    const c10::DeviceGuard guard(first.device());
    const SourceTable table = source_table(sources);
    const Tensor grad_out = grads[0].to(torch::kBFloat16).contiguous();
    const Tensor out = save ? saved[S + 2].contiguous() : Tensor();
    const StatePointers state = pool_pointers(saved[S + 1], pool_layout(N, S, D, save), save);
    std::vector<Tensor> dv;
    std::vector<void*> dv_rows;
    dv.reserve(S);
    dv_rows.reserve(S);
    for (int64_t s = 0; s < S; ++s) {
      dv.push_back(bf16_empty(first.sizes(), first));
      dv_rows.push_back(dv.back().data_ptr());
    }
    Tensor grad_query = bf16_empty({R}, first);
    Tensor workspace = dq_workspace(N, D, R, first);
    check(attnres_hip_sources_backward(table.rows.data(), table.strides.data(), S, N, D, query.data_ptr(), R,
                                       static_cast<float>(ctx->saved_data["scale"].toDouble()),
                                       save ? out.data_ptr() : nullptr, state.refine, grad_out.data_ptr(), state.logit,
                                       state.inv_rms, state.stats, dv_rows.data(), grad_query.data_ptr(),
                                       workspace.data_ptr<float>(), workspace.numel(), current_stream(first)),
          "attnres source-list backward");
    if (ctx->needs_input_grad(0)) result[0] = grad_query;
    for (int64_t s = 0; s < S; ++s) {
      if (ctx->needs_input_grad(1 + s)) result[3 + s] = dv[s];
    }
    return result;
  }
};

// ------------------------------------------------------ no gradient needed

// Grad mode off (torch.no_grad, inference_mode) or no input requiring grad:
// no node, no saved state and no refinement bytes (the forward takes
// out_refine = NULL for any S); the statistics the kernels write go to a
// scratch allocation freed on return.  out is the same, bit for bit.
bool needs_grad(const Tensor& query, at::TensorList sources) {
  if (!at::GradMode::is_enabled()) return false;
  if (query.requires_grad()) return true;
  for (const Tensor& source : sources) {
    if (source.requires_grad()) return true;
  }
  return false;
}

Tensor statistics_scratch(int64_t tokens, int64_t sources, const Tensor& like, StatePointers* state) {
  const PoolLayout layout = pool_layout(tokens, sources, 0, false);
  Tensor pool = torch::empty({layout.size}, like.options().dtype(torch::kUInt8));
  *state = pool_pointers(pool, layout, false);
  return pool;
}

Tensor packed_forward_only(const Tensor& values, const Tensor& query, double eps, double scale) {
  const int64_t S = values.size(0), D = values.size(-1), R = query.numel();
  const Tensor rows = flat_rows(values);
  const int64_t N = rows.size(1);
  const c10::DeviceGuard guard(values.device());
  Tensor out = bf16_empty(values.sizes().slice(1), values);
  StatePointers state{};
  const Tensor scratch = statistics_scratch(N, S, values, &state);
  check(attnres_hip_packed_forward(rows.data_ptr(), rows.stride(0), rows.stride(1), S, N, D, query.data_ptr(), R,
                                   static_cast<float>(eps), static_cast<float>(scale), out.data_ptr(), nullptr,
                                   state.logit, state.inv_rms, state.stats, current_stream(values)),
        "attnres packed forward");
  return out;
}

Tensor sources_forward_only(const Tensor& query, double eps, double scale, at::TensorList sources) {
  const Tensor& first = sources[0];
  const int64_t S = static_cast<int64_t>(sources.size()), N = rows_of(first), D = first.size(-1);
  const c10::DeviceGuard guard(first.device());
  const SourceTable table = source_table(sources);
  Tensor out = bf16_empty(first.sizes(), first);
  StatePointers state{};
  const Tensor scratch = statistics_scratch(N, S, first, &state);
  check(attnres_hip_sources_forward(table.rows.data(), table.strides.data(), S, N, D, query.data_ptr(),
                                    query.numel(), static_cast<float>(eps), static_cast<float>(scale),
                                    out.data_ptr(), nullptr, state.logit, state.inv_rms, state.stats,
                                    current_stream(first)),
        "attnres source-list forward");
  return out;
}

Tensor packed_read(const Tensor& values, const Tensor& query, double eps, double scale) {
  if (!needs_grad(query, values)) return packed_forward_only(values, query, eps, scale);
  return PackedRead::apply(values, query, eps, scale);
}

Tensor sources_read(const Tensor& query, double eps, double scale, const std::vector<Tensor>& sources) {
  if (!needs_grad(query, sources)) return sources_forward_only(query, eps, scale, sources);
  return SourcesRead::apply(query, eps, scale, at::TensorList(sources));
}

std::tuple<int64_t, int64_t, int64_t> layout_of(int64_t tokens, int64_t sources, int64_t width, bool save) {
  const PoolLayout layout = pool_layout(tokens, sources, width, save);
  return {layout.head, layout.block, layout.size};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Eager autograd nodes of the attnres read over the attnres_hip C ABI";
  m.def("packed_read", &packed_read, "packed read [S, ..., D] (eager autograd node)");
  m.def("sources_read", &sources_read, "source-list read (eager autograd node)");
  m.def("pool_layout", &layout_of, "(head, block, size) of the pooled saved state");
}
