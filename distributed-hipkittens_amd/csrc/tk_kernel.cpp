// pybind11 module `tk_kernel`: the Python-callable dispatch_* entry points of
// the FP8 MoE path, layered over the C ABI in include/hkmoe.h.
//
// Mirrors the reference's binding convention (include/pyutils/pyutils.cuh):
// positional torch.Tensor arguments, each checked to be a Tensor
// (class-name check), contiguous and not on the CPU (pyutils.cuh:17-26), with
// failures raised as RuntimeError; `dispatch_micro(A, B, C)` keeps the
// reference's dense-GEMM call (kernels/cdna3/gemm/fp8fp32/mi300x/
// 8192_256_256_64_32/data_logs/0613_003858_outputs/256_256_64_32.cpp:202-212).
// Additions over the reference: dtype and shape checks, and launches go to
// torch's current stream of the current device instead of the null stream.
//
// No torch C++ headers: tensors are read through their Python attributes, so
// this module only depends on pybind11 and the C ABI.
#include <pybind11/pybind11.h>

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/hkmoe.h"

namespace py = pybind11;

namespace {

struct TensorArg {
  void* ptr = nullptr;
  std::vector<int64_t> shape;
  std::string dtype;
  int64_t numel() const {
    int64_t n = 1;
    for (auto s : shape) n *= s;
    return n;
  }
};

TensorArg as_tensor(const py::object& obj, const char* name) {
  if (!py::hasattr(obj, "__class__") ||
      obj.attr("__class__").attr("__name__").cast<std::string>() != "Tensor")
    throw std::runtime_error(std::string(name) + ": expected a torch.Tensor");
  if (!obj.attr("is_contiguous")().cast<bool>())
    throw std::runtime_error(std::string(name) + ": tensor must be contiguous");
  if (obj.attr("device").attr("type").cast<std::string>() == "cpu")
    throw std::runtime_error(std::string(name) + ": tensor must be on a GPU device");
  TensorArg t;
  t.ptr = reinterpret_cast<void*>(obj.attr("data_ptr")().cast<uintptr_t>());
  for (auto s : obj.attr("shape").cast<py::tuple>()) t.shape.push_back(s.cast<int64_t>());
  t.dtype = py::str(obj.attr("dtype")).cast<std::string>();
  return t;
}

TensorArg as_tensor_opt(const py::object& obj, const char* name) {
  if (obj.is_none()) return TensorArg{};
  return as_tensor(obj, name);
}

void want_dtype(const TensorArg& t, const char* name, const char* dtype) {
  if (t.ptr != nullptr && t.dtype != dtype)
    throw std::runtime_error(std::string(name) + ": expected dtype " + dtype + ", got " + t.dtype);
}

void want_dim(const TensorArg& t, const char* name, size_t nd) {
  if (t.shape.size() != nd)
    throw std::runtime_error(std::string(name) + ": expected " + std::to_string(nd) + "-D tensor");
}

hkmoe_stream_t current_stream() {
  // Intentionally leaked: a static py::object would be destroyed after the
  // interpreter has finalised and crash the process at exit.
  static py::object* torch_cuda = new py::object(py::module_::import("torch").attr("cuda"));
  const uintptr_t s = torch_cuda->attr("current_stream")().attr("cuda_stream").cast<uintptr_t>();
  return reinterpret_cast<hkmoe_stream_t>(s);
}

void check(int rc) {
  if (rc != HKMOE_OK) throw std::runtime_error(std::string("hkmoe: ") + hkmoe_last_error());
}

constexpr const char* kF8 = "torch.float8_e4m3fn";
constexpr const char* kBf16 = "torch.bfloat16";
constexpr const char* kF32 = "torch.float32";
constexpr const char* kI32 = "torch.int32";

int scale_mode_of(const TensorArg& s) {
  return (s.shape.size() <= 1 && s.numel() == 1) ? HKMOE_SCALE_TENSOR : HKMOE_SCALE_BLOCK;
}

// ---------------------------------------------------------------------------

void dispatch_gemm(py::object A, py::object B, py::object C, py::object sa, py::object sb) {
  auto a = as_tensor(A, "A"), b = as_tensor(B, "B"), c = as_tensor(C, "C");
  auto as = as_tensor_opt(sa, "scale_a"), bs = as_tensor_opt(sb, "scale_b");
  want_dtype(a, "A", kF8);
  want_dtype(b, "B", kF8);
  want_dtype(as, "scale_a", kF32);
  want_dtype(bs, "scale_b", kF32);
  // Like gl<> views (pyutils.cuh:28-38), leading size-1 dims are ignored.
  auto rows_cols = [](const TensorArg& t, const char* n) {
    if (t.shape.size() < 2 || t.shape.size() > 4) throw std::runtime_error(std::string(n) + ": expected 2-4 dims");
    for (size_t i = 0; i + 2 < t.shape.size(); ++i)
      if (t.shape[i] != 1) throw std::runtime_error(std::string(n) + ": leading dims must be 1");
    return std::pair<int64_t, int64_t>(t.shape[t.shape.size() - 2], t.shape.back());
  };
  auto [m, k] = rows_cols(a, "A");
  auto [n, kb] = rows_cols(b, "B");
  auto [cm, cn] = rows_cols(c, "C");
  if (k != kb) throw std::runtime_error("A and B must have the same K");
  if (cm != m || cn != n) throw std::runtime_error("C must be [M, N]");
  if (as.ptr && as.numel() != 1) throw std::runtime_error("scale_a must hold one value");
  if (bs.ptr && bs.numel() != 1) throw std::runtime_error("scale_b must hold one value");
  int out;
  if (c.dtype == kBf16) out = HKMOE_BF16;
  else if (c.dtype == kF32) out = HKMOE_F32;
  else throw std::runtime_error("C: expected bfloat16 or float32");
  check(hkmoe_gemm_fp8(a.ptr, b.ptr, c.ptr, m, n, k, static_cast<const float*>(as.ptr),
                       static_cast<const float*>(bs.ptr), out, current_stream()));
}

void dispatch_micro(py::object A, py::object B, py::object C) {
  dispatch_gemm(A, B, C, py::none(), py::none());
}

void dispatch_route_topk(py::object logits, py::object idx, py::object w, py::object bc) {
  auto l = as_tensor(logits, "logits"), i = as_tensor(idx, "topk_idx"), ww = as_tensor(w, "topk_w"),
       b = as_tensor(bc, "block_counts");
  want_dtype(l, "logits", kF32);
  want_dtype(i, "topk_idx", kI32);
  want_dtype(ww, "topk_w", kF32);
  want_dtype(b, "block_counts", kI32);
  want_dim(l, "logits", 2);
  want_dim(i, "topk_idx", 2);
  const int64_t t = l.shape[0], e = l.shape[1], k = i.shape[1];
  if (i.shape[0] != t || ww.shape != i.shape) throw std::runtime_error("topk_idx/topk_w must be [T, k]");
  if (b.numel() < static_cast<int64_t>(hkmoe_route_blocks(t)) * e)
    throw std::runtime_error("block_counts too small: need route_blocks(T) * E");
  check(hkmoe_route_topk(static_cast<const float*>(l.ptr), t, static_cast<int32_t>(e),
                         static_cast<int32_t>(k), static_cast<int32_t*>(i.ptr),
                         static_cast<float*>(ww.ptr), static_cast<int32_t*>(b.ptr), current_stream()));
}

// Upper bound of the M tiles of T tokens over E experts (top-k <= min(E, 32)).
int64_t mtile_list_ints(int64_t rows, int64_t e) { return 2 * ((rows + 255) / 256 + e); }

void dispatch_expert_offsets(py::object bc, int64_t num_tokens, py::object counts, py::object offsets,
                             py::object block_base, py::object mtile_offsets, py::object amax,
                             py::object tile_counters, py::object mtile_list, int32_t narrow_max,
                             py::object narrow_info) {
  auto ni = as_tensor_opt(narrow_info, "narrow_info");
  want_dtype(ni, "narrow_info", kI32);
  if (ni.ptr && ni.numel() < 5) throw std::runtime_error("narrow_info must hold 5 ints");
  auto b = as_tensor(bc, "block_counts"), c = as_tensor(counts, "counts"),
       o = as_tensor(offsets, "offsets"), bb = as_tensor(block_base, "block_base"),
       mo = as_tensor(mtile_offsets, "mtile_offsets"), am = as_tensor_opt(amax, "amax"),
       tc = as_tensor_opt(tile_counters, "tile_counters"), ml = as_tensor_opt(mtile_list, "mtile_list");
  want_dtype(ml, "mtile_list", kI32);
  for (auto* t : {&b, &c, &o, &bb, &mo}) want_dtype(*t, "int tensor", kI32);
  want_dtype(am, "amax", kF32);
  want_dtype(tc, "tile_counters", kI32);
  if (tc.ptr && tc.numel() < HKMOE_TILE_COUNTERS) throw std::runtime_error("tile_counters must hold 16 ints");
  const int64_t e = c.numel();
  if (o.numel() != e + 1 || mo.numel() != e + 1) throw std::runtime_error("offsets must hold E+1 values");
  if (b.numel() < static_cast<int64_t>(hkmoe_route_blocks(num_tokens)) * e || bb.numel() < b.numel())
    throw std::runtime_error("block_counts/block_base too small");
  if (ml.ptr && ml.numel() < mtile_list_ints(num_tokens * std::min<int64_t>(e, 32), e))
    throw std::runtime_error("mtile_list must hold 2 * (ceil(T * min(E, 32) / 256) + E) ints");
  if (ni.ptr) {
    check(hkmoe_expert_offsets_narrow(static_cast<const int32_t*>(b.ptr), num_tokens, static_cast<int32_t>(e),
                                      static_cast<int32_t*>(c.ptr), static_cast<int32_t*>(o.ptr),
                                      static_cast<int32_t*>(bb.ptr), static_cast<int32_t*>(mo.ptr),
                                      static_cast<int32_t*>(ml.ptr), static_cast<float*>(am.ptr),
                                      static_cast<int32_t*>(tc.ptr), narrow_max, static_cast<int32_t*>(ni.ptr),
                                      current_stream()));
    return;
  }
  check(hkmoe_expert_offsets(static_cast<const int32_t*>(b.ptr), num_tokens, static_cast<int32_t>(e),
                             static_cast<int32_t*>(c.ptr), static_cast<int32_t*>(o.ptr),
                             static_cast<int32_t*>(bb.ptr), static_cast<int32_t*>(mo.ptr),
                             static_cast<int32_t*>(ml.ptr), static_cast<float*>(am.ptr),
                             static_cast<int32_t*>(tc.ptr), current_stream()));
}

void dispatch_scatter(py::object idx, py::object offsets, py::object block_base, py::object perm,
                      py::object inv_perm, py::object x_q, py::object x_scale, py::object xp,
                      py::object xps_t) {
  auto i = as_tensor(idx, "topk_idx"), o = as_tensor(offsets, "offsets"),
       bb = as_tensor(block_base, "block_base"), p = as_tensor(perm, "perm"),
       ip = as_tensor(inv_perm, "inv_perm"), x = as_tensor_opt(x_q, "x_q"),
       xs = as_tensor_opt(x_scale, "x_scale"), d = as_tensor_opt(xp, "xp"),
       ds = as_tensor_opt(xps_t, "xp_scale_t");
  want_dim(i, "topk_idx", 2);
  for (auto* t : {&i, &o, &bb, &p, &ip}) want_dtype(*t, "int tensor", kI32);
  want_dtype(x, "x_q", kF8);
  want_dtype(d, "xp", kF8);
  want_dtype(xs, "x_scale", kF32);
  want_dtype(ds, "xp_scale_t", kF32);
  const int64_t t = i.shape[0], k = i.shape[1], e = o.numel() - 1;
  if (p.numel() != t * k || ip.numel() != t * k) throw std::runtime_error("perm/inv_perm must hold T*k values");
  int64_t hidden = 0;
  int mode = HKMOE_SCALE_TENSOR;
  if (x.ptr) {
    want_dim(x, "x_q", 2);
    hidden = x.shape[1];
    if (x.shape[0] != t) throw std::runtime_error("x_q must be [T, H]");
    if ((t > 0 && !d.ptr) || d.numel() != t * k * hidden) throw std::runtime_error("xp must be [T*k, H]");
    if (ds.ptr) {
      mode = HKMOE_SCALE_BLOCK;
      if ((t > 0 && !xs.ptr) || xs.numel() != t * (hidden / 128) || ds.numel() != t * k * (hidden / 128))
        throw std::runtime_error("block scales: x_scale [T, H/128], xp_scale_t [H/128, T*k]");
    }
  }
  check(hkmoe_scatter(static_cast<const int32_t*>(i.ptr), t, static_cast<int32_t>(e),
                      static_cast<int32_t>(k), static_cast<const int32_t*>(o.ptr),
                      static_cast<const int32_t*>(bb.ptr), static_cast<int32_t*>(p.ptr),
                      static_cast<int32_t*>(ip.ptr), x.ptr, static_cast<const float*>(xs.ptr), hidden,
                      mode, d.ptr, static_cast<float*>(ds.ptr), current_stream()));
}

void dispatch_grouped_gemm1(py::object x_q, py::object x_scale, py::object gather, int32_t gather_div,
                            py::object w13, py::object w13s, py::object offsets, py::object mtile_offsets,
                            py::object h, py::object h_aux, py::object tile_counters, bool packed,
                            py::object mtile_list, py::object narrow_info, int32_t part, int32_t grid) {
  auto ni = as_tensor_opt(narrow_info, "narrow_info");
  want_dtype(ni, "narrow_info", kI32);
  auto x = as_tensor(x_q, "x"), xs = as_tensor(x_scale, "x_scale"), gth = as_tensor_opt(gather, "gather"),
       w = as_tensor(w13, "w13"), ws = as_tensor(w13s, "w13_scale"), o = as_tensor(offsets, "offsets"),
       mo = as_tensor(mtile_offsets, "mtile_offsets"), hh = as_tensor(h, "h"),
       aux = as_tensor_opt(h_aux, "h_aux"), tc = as_tensor_opt(tile_counters, "tile_counters"),
       ml = as_tensor_opt(mtile_list, "mtile_list");
  want_dtype(tc, "tile_counters", kI32);
  want_dtype(ml, "mtile_list", kI32);
  if (tc.ptr && tc.numel() < 8) throw std::runtime_error("tile_counters must hold 8 ints");
  want_dtype(x, "x", kF8);
  want_dtype(w, "w13", kF8);
  want_dtype(xs, "x_scale", kF32);
  want_dtype(ws, "w13_scale", kF32);
  want_dtype(gth, "gather", kI32);
  want_dtype(aux, "h_aux", kF32);
  want_dim(x, "x", 2);
  want_dim(w, "w13", 3);
  want_dim(hh, "h", 2);
  const int64_t x_rows = x.shape[0], hidden = x.shape[1], e = w.shape[0], inter = w.shape[1] / 2;
  const int64_t rows = hh.shape[0];
  if (w.shape[2] != hidden || w.shape[1] % 2) throw std::runtime_error("w13 must be [E, 2I, H]");
  if (hh.shape[1] != inter) throw std::runtime_error("h must be [rows, I]");
  if (gth.ptr && gth.numel() != rows) throw std::runtime_error("gather must hold one index per row");
  if (ml.ptr && ml.numel() < mtile_list_ints(rows, e)) throw std::runtime_error("mtile_list too small");
  if (o.numel() != e + 1 || mo.numel() != e + 1) throw std::runtime_error("offsets must hold E+1 values");
  int fmt;
  if (hh.dtype == kBf16) fmt = HKMOE_BF16;
  else if (hh.dtype == kF8) fmt = HKMOE_E4M3;
  else throw std::runtime_error("h: expected bfloat16 or float8_e4m3fn");
  const int mode = scale_mode_of(xs);
  if (mode == HKMOE_SCALE_TENSOR && ws.numel() != e) throw std::runtime_error("w13_scale must be [E]");
  if (mode == HKMOE_SCALE_BLOCK &&
      (xs.numel() != x_rows * (hidden / 128) || ws.numel() != e * (2 * inter / 128) * (hidden / 128)))
    throw std::runtime_error("block scales: x_scale [x_rows, H/128], w13_scale [E, 2I/128, H/128]");
  if (fmt == HKMOE_E4M3 && ((rows > 0 && !aux.ptr) || aux.numel() != rows * (inter / 128)))
    throw std::runtime_error("e4m3 output needs h_aux [I/128, rows] group scales");
  if (ni.ptr) {
    if (mode != HKMOE_SCALE_BLOCK || fmt != HKMOE_E4M3 || !ml.ptr)
      throw std::runtime_error("narrow split: needs block scales, e4m3 h and the M-tile list");
    check(hkmoe_grouped_gemm1_part(x.ptr, static_cast<const float*>(xs.ptr), static_cast<const int32_t*>(gth.ptr),
                                   gather_div, x_rows, w.ptr, static_cast<const float*>(ws.ptr),
                                   static_cast<const int32_t*>(o.ptr), static_cast<const int32_t*>(mo.ptr),
                                   static_cast<const int32_t*>(ml.ptr), rows, static_cast<int32_t>(e),
                                   static_cast<int32_t>(hidden), static_cast<int32_t>(inter),
                                   packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, hh.ptr, static_cast<float*>(aux.ptr),
                                   static_cast<int32_t*>(tc.ptr), static_cast<const int32_t*>(ni.ptr), part, grid,
                                   current_stream()));
    return;
  }
  check(hkmoe_grouped_gemm1(x.ptr, static_cast<const float*>(xs.ptr), static_cast<const int32_t*>(gth.ptr),
                            gather_div, x_rows, w.ptr, static_cast<const float*>(ws.ptr),
                            static_cast<const int32_t*>(o.ptr), static_cast<const int32_t*>(mo.ptr),
                            static_cast<const int32_t*>(ml.ptr), rows,
                            static_cast<int32_t>(e), static_cast<int32_t>(hidden), static_cast<int32_t>(inter),
                            mode, packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, fmt, hh.ptr,
                            static_cast<float*>(aux.ptr), static_cast<int32_t*>(tc.ptr), current_stream()));
}

// counts [2] int32 (zeroed by the caller) += (cases, mismatches) of the
// requantisation-quotient self-check (hkmoe_requant_quotient_check)
void dispatch_requant_quotient_check(py::object counts) {
  auto c = as_tensor(counts, "counts");
  want_dtype(c, "counts", kI32);
  if (c.numel() != 2) throw std::runtime_error("counts must hold two int32");
  check(hkmoe_requant_quotient_check(static_cast<int32_t*>(c.ptr), current_stream()));
}

void dispatch_requant(py::object h, py::object amax, py::object hq, py::object hs) {
  auto hh = as_tensor(h, "h"), am = as_tensor_opt(amax, "amax"), q = as_tensor(hq, "hq"),
       s = as_tensor(hs, "hs");
  want_dtype(hh, "h", kBf16);
  want_dtype(q, "hq", kF8);
  want_dtype(s, "hs", kF32);
  want_dtype(am, "amax", kF32);
  want_dim(hh, "h", 2);
  const int64_t rows = hh.shape[0], inter = hh.shape[1];
  if (q.numel() != rows * inter) throw std::runtime_error("hq must be [rows, I]");
  // per-tensor mode iff GEMM 1's running amax is supplied
  const int mode = am.ptr ? HKMOE_SCALE_TENSOR : HKMOE_SCALE_BLOCK;
  if (mode == HKMOE_SCALE_TENSOR && s.numel() != 1) throw std::runtime_error("hs must hold one value");
  if (mode == HKMOE_SCALE_BLOCK && s.numel() != rows * (inter / 128))
    throw std::runtime_error("hs must be [I/128, rows] for group scales");
  check(hkmoe_requant(hh.ptr, rows, static_cast<int32_t>(inter), mode, static_cast<const float*>(am.ptr),
                      q.ptr, static_cast<float*>(s.ptr), current_stream()));
}

void dispatch_grouped_gemm2(py::object hq, py::object hs, py::object w2, py::object w2s,
                            py::object offsets, py::object mtile_offsets, py::object y,
                            py::object tile_counters, bool packed, py::object mtile_list,
                            py::object narrow_info, int32_t part, int32_t grid) {
  auto ni = as_tensor_opt(narrow_info, "narrow_info");
  want_dtype(ni, "narrow_info", kI32);
  auto q = as_tensor(hq, "hq"), s = as_tensor(hs, "hs"), w = as_tensor(w2, "w2"),
       ws = as_tensor(w2s, "w2_scale"), o = as_tensor(offsets, "offsets"),
       mo = as_tensor(mtile_offsets, "mtile_offsets"), yy = as_tensor(y, "y"),
       tc = as_tensor_opt(tile_counters, "tile_counters"), ml = as_tensor_opt(mtile_list, "mtile_list");
  want_dtype(tc, "tile_counters", kI32);
  want_dtype(ml, "mtile_list", kI32);
  if (tc.ptr && tc.numel() < 8) throw std::runtime_error("tile_counters must hold 8 ints");
  want_dtype(q, "hq", kF8);
  want_dtype(w, "w2", kF8);
  want_dtype(s, "hs", kF32);
  want_dtype(ws, "w2_scale", kF32);
  want_dtype(yy, "y", kBf16);
  want_dim(q, "hq", 2);
  want_dim(w, "w2", 3);
  const int64_t rows = q.shape[0], inter = q.shape[1], e = w.shape[0], hidden = w.shape[1];
  if (w.shape[2] != inter) throw std::runtime_error("w2 must be [E, H, I]");
  if (yy.numel() != rows * hidden) throw std::runtime_error("y must be [rows, H]");
  if (o.numel() != e + 1 || mo.numel() != e + 1) throw std::runtime_error("offsets must hold E+1 values");
  if (ml.ptr && ml.numel() < mtile_list_ints(rows, e)) throw std::runtime_error("mtile_list too small");
  const int mode = scale_mode_of(s);
  if (mode == HKMOE_SCALE_TENSOR && ws.numel() != e) throw std::runtime_error("w2_scale must be [E]");
  if (mode == HKMOE_SCALE_BLOCK &&
      (s.numel() != rows * (inter / 128) || ws.numel() != e * (hidden / 128) * (inter / 128)))
    throw std::runtime_error("block scales: hs [I/128, rows], w2_scale [E, H/128, I/128]");
  if (ni.ptr) {
    if (mode != HKMOE_SCALE_BLOCK || !ml.ptr)
      throw std::runtime_error("narrow split: needs block scales and the M-tile list");
    check(hkmoe_grouped_gemm2_part(q.ptr, static_cast<const float*>(s.ptr), w.ptr,
                                   static_cast<const float*>(ws.ptr), static_cast<const int32_t*>(o.ptr),
                                   static_cast<const int32_t*>(mo.ptr), static_cast<const int32_t*>(ml.ptr), rows,
                                   static_cast<int32_t>(e), static_cast<int32_t>(hidden),
                                   static_cast<int32_t>(inter), packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, yy.ptr,
                                   static_cast<int32_t*>(tc.ptr), static_cast<const int32_t*>(ni.ptr), part, grid,
                                   current_stream()));
    return;
  }
  check(hkmoe_grouped_gemm2(q.ptr, static_cast<const float*>(s.ptr), w.ptr,
                            static_cast<const float*>(ws.ptr), static_cast<const int32_t*>(o.ptr),
                            static_cast<const int32_t*>(mo.ptr), static_cast<const int32_t*>(ml.ptr), rows,
                            static_cast<int32_t>(e),
                            static_cast<int32_t>(hidden), static_cast<int32_t>(inter), mode,
                            packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, yy.ptr, static_cast<int32_t*>(tc.ptr),
                            current_stream()));
}

void dispatch_combine(py::object y, py::object w, py::object inv_perm, py::object out) {
  auto yy = as_tensor(y, "y"), ww = as_tensor(w, "topk_w"), ip = as_tensor(inv_perm, "inv_perm"),
       o = as_tensor(out, "out");
  want_dtype(yy, "y", kBf16);
  want_dtype(ww, "topk_w", kF32);
  want_dtype(ip, "inv_perm", kI32);
  want_dtype(o, "out", kBf16);
  want_dim(ww, "topk_w", 2);
  want_dim(o, "out", 2);
  const int64_t t = ww.shape[0], k = ww.shape[1], hidden = o.shape[1];
  if (o.shape[0] != t || yy.numel() != t * k * hidden || ip.numel() != t * k)
    throw std::runtime_error("combine: y [T*k, H], inv_perm [T*k], out [T, H]");
  check(hkmoe_combine(yy.ptr, static_cast<const float*>(ww.ptr), static_cast<const int32_t*>(ip.ptr), t,
                      static_cast<int32_t>(k), static_cast<int32_t>(hidden), o.ptr, current_stream()));
}

size_t moe_workspace_size(int64_t t, int32_t e, int32_t k, int32_t hidden, int32_t inter, int mode) {
  return hkmoe_moe_workspace_size(t, e, k, hidden, inter, mode);
}

void dispatch_moe(py::object x_q, py::object x_scale, py::object logits, py::object w13,
                  py::object w13s, py::object w2, py::object w2s, int32_t top_k, py::object out,
                  py::object workspace, bool packed) {
  auto x = as_tensor(x_q, "x_q"), xs = as_tensor(x_scale, "x_scale"), l = as_tensor(logits, "logits"),
       a = as_tensor(w13, "w13"), as = as_tensor(w13s, "w13_scale"), b = as_tensor(w2, "w2"),
       bs = as_tensor(w2s, "w2_scale"), o = as_tensor(out, "out"), ws = as_tensor(workspace, "workspace");
  want_dtype(x, "x_q", kF8);
  want_dtype(a, "w13", kF8);
  want_dtype(b, "w2", kF8);
  for (auto* t : {&xs, &l, &as, &bs}) want_dtype(*t, "fp32 tensor", kF32);
  want_dtype(o, "out", kBf16);
  want_dim(x, "x_q", 2);
  want_dim(l, "logits", 2);
  want_dim(a, "w13", 3);
  want_dim(b, "w2", 3);
  const int64_t t = x.shape[0], hidden = x.shape[1], e = a.shape[0], inter = a.shape[1] / 2;
  if (l.shape[0] != t || l.shape[1] != e) throw std::runtime_error("logits must be [T, E]");
  if (a.shape[2] != hidden || b.shape[0] != e || b.shape[1] != hidden || b.shape[2] != inter)
    throw std::runtime_error("w13 must be [E, 2I, H] and w2 [E, H, I]");
  if (o.numel() != t * hidden) throw std::runtime_error("out must be [T, H]");
  const int mode = scale_mode_of(xs);
  if (mode == HKMOE_SCALE_BLOCK &&
      (xs.numel() != t * (hidden / 128) || as.numel() != e * (2 * inter / 128) * (hidden / 128) ||
       bs.numel() != e * (hidden / 128) * (inter / 128)))
    throw std::runtime_error("block scales: x_scale [T, H/128], w13_scale [E, 2I/128, H/128], w2_scale [E, H/128, I/128]");
  if (mode == HKMOE_SCALE_TENSOR && (as.numel() != e || bs.numel() != e))
    throw std::runtime_error("per-tensor scales: w13_scale and w2_scale must be [E]");
  const size_t bytes = static_cast<size_t>(ws.numel()) * (ws.dtype == kF32 || ws.dtype == kI32 ? 4 : 1);
  check(hkmoe_moe_forward(x.ptr, static_cast<const float*>(xs.ptr), static_cast<const float*>(l.ptr), a.ptr,
                          static_cast<const float*>(as.ptr), b.ptr, static_cast<const float*>(bs.ptr), t,
                          static_cast<int32_t>(e), top_k, static_cast<int32_t>(hidden),
                          static_cast<int32_t>(inter), mode, packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, o.ptr,
                          ws.ptr, bytes, current_stream()));
}

// Load-time packing of expert weights [E, N, K] into the grouped GEMMs' tile
// layout (same shape and size; pass packed=True to the GEMMs afterwards).
void dispatch_pack_weights(py::object w, py::object packed, int32_t gate_up) {
  auto src = as_tensor(w, "w"), dst = as_tensor(packed, "packed");
  want_dtype(src, "w", kF8);
  want_dtype(dst, "packed", kF8);
  want_dim(src, "w", 3);
  if (dst.shape != src.shape) throw std::runtime_error("packed must have the shape of w");
  check(hkmoe_pack_weights(src.ptr, src.shape[0], src.shape[1], src.shape[2], gate_up, dst.ptr,
                           current_stream()));
}

void dispatch_quant_group(py::object x, py::object q, py::object s) {
  auto xx = as_tensor(x, "x"), qq = as_tensor(q, "q"), ss = as_tensor(s, "s");
  want_dtype(xx, "x", kF32);
  want_dtype(qq, "q", kF8);
  want_dtype(ss, "s", kF32);
  want_dim(xx, "x", 2);
  const int64_t r = xx.shape[0], c = xx.shape[1];
  if (qq.numel() != r * c || ss.numel() != r * (c / 128)) throw std::runtime_error("quant_group: q [R,C], s [R,C/128]");
  check(hkmoe_quant_group(static_cast<const float*>(xx.ptr), r, c, qq.ptr, static_cast<float*>(ss.ptr),
                          current_stream()));
}

void dispatch_quant_block(py::object x, py::object q, py::object s) {
  auto xx = as_tensor(x, "x"), qq = as_tensor(q, "q"), ss = as_tensor(s, "s");
  want_dtype(xx, "x", kF32);
  want_dtype(qq, "q", kF8);
  want_dtype(ss, "s", kF32);
  if (xx.shape.size() != 2 && xx.shape.size() != 3) throw std::runtime_error("quant_block: x must be 2-D or 3-D");
  const int64_t b = xx.shape.size() == 3 ? xx.shape[0] : 1;
  const int64_t r = xx.shape[xx.shape.size() - 2], c = xx.shape.back();
  if (qq.numel() != b * r * c || ss.numel() != b * (r / 128) * (c / 128))
    throw std::runtime_error("quant_block: q like x, s [B, R/128, C/128]");
  check(hkmoe_quant_block(static_cast<const float*>(xx.ptr), b, r, c, qq.ptr, static_cast<float*>(ss.ptr),
                          current_stream()));
}

void dispatch_quant_tensor(py::object x, py::object q, py::object s, py::object ws) {
  auto xx = as_tensor(x, "x"), qq = as_tensor(q, "q"), ss = as_tensor(s, "s"), w = as_tensor(ws, "amax_ws");
  want_dtype(xx, "x", kF32);
  want_dtype(qq, "q", kF8);
  want_dtype(ss, "s", kF32);
  want_dtype(w, "amax_ws", kF32);
  if (qq.numel() != xx.numel() || ss.numel() != 1 || w.numel() < 1)
    throw std::runtime_error("quant_tensor: q like x, s [1], amax_ws [1]");
  check(hkmoe_quant_tensor(static_cast<const float*>(xx.ptr), 1, xx.numel(), qq.ptr,
                           static_cast<float*>(ss.ptr), static_cast<float*>(w.ptr), current_stream()));
}

// MX (e8m0 1x32) operands: raw exponents are uint8 [R, C/32]; packed
// exponent words are int32 [C/128, R64] (R64 = R rounded up to 64).
constexpr const char* kU8 = "torch.uint8";

int64_t round64(int64_t r) { return (r + 63) / 64 * 64; }

void dispatch_quant_mx(py::object x, py::object q, py::object s) {
  auto xx = as_tensor(x, "x"), qq = as_tensor(q, "q"), ss = as_tensor(s, "s");
  want_dtype(xx, "x", kF32);
  want_dtype(qq, "q", kF8);
  want_dtype(ss, "s", kU8);
  want_dim(xx, "x", 2);
  const int64_t r = xx.shape[0], c = xx.shape[1];
  if (qq.numel() != r * c || ss.numel() != r * (c / 32)) throw std::runtime_error("quant_mx: q [R,C], s [R,C/32]");
  check(hkmoe_quant_mx(static_cast<const float*>(xx.ptr), r, c, qq.ptr, ss.ptr, current_stream()));
}

void dispatch_mx_pack_scales(py::object s, int64_t cols, py::object packed) {
  auto ss = as_tensor(s, "s"), pp = as_tensor(packed, "packed");
  want_dtype(ss, "s", kU8);
  want_dtype(pp, "packed", kI32);
  want_dim(ss, "s", 2);
  const int64_t r = ss.shape[0];
  if (cols % 128 != 0 || ss.shape[1] != cols / 32)
    throw std::runtime_error("mx_pack_scales: s must be [R, cols/32] with cols % 128 == 0");
  if (pp.numel() != (cols / 128) * round64(r)) throw std::runtime_error("mx_pack_scales: packed must be [cols/128, R64]");
  check(hkmoe_mx_pack_scales(ss.ptr, r, cols, pp.ptr, current_stream()));
}

void dispatch_gemm_mx(py::object A, py::object sa, py::object B, py::object sb, py::object C) {
  auto a = as_tensor(A, "A"), b = as_tensor(B, "B"), c = as_tensor(C, "C");
  auto as = as_tensor(sa, "scale_a"), bs = as_tensor(sb, "scale_b");
  want_dtype(a, "A", kF8);
  want_dtype(b, "B", kF8);
  want_dtype(as, "scale_a", kI32);
  want_dtype(bs, "scale_b", kI32);
  want_dim(a, "A", 2);
  want_dim(b, "B", 2);
  want_dim(c, "C", 2);
  const int64_t m = a.shape[0], k = a.shape[1], n = b.shape[0];
  if (b.shape[1] != k) throw std::runtime_error("A and B must have the same K");
  if (c.shape[0] != m || c.shape[1] != n) throw std::runtime_error("C must be [M, N]");
  if (as.numel() != (k / 128) * round64(m)) throw std::runtime_error("scale_a must be packed [K/128, M64]");
  if (bs.numel() != (k / 128) * round64(n)) throw std::runtime_error("scale_b must be packed [K/128, N]");
  int out;
  if (c.dtype == kBf16) out = HKMOE_BF16;
  else if (c.dtype == kF32) out = HKMOE_F32;
  else throw std::runtime_error("C: expected bfloat16 or float32");
  check(hkmoe_gemm_mx(a.ptr, as.ptr, b.ptr, bs.ptr, c.ptr, m, n, k, out, current_stream()));
}

// MX MoE layer: e8m0 bytes are uint8 tensors, packed exponent words int32.
int64_t mx_ws(int64_t rows, int64_t e) { return hkmoe_mx_words_per_step(rows, static_cast<int32_t>(e)); }

void dispatch_mx_pack_weight_scales(py::object s, py::object words, int32_t gate_up) {
  auto ss = as_tensor(s, "s"), ww = as_tensor(words, "words");
  want_dtype(ss, "s", kU8);
  want_dtype(ww, "words", kI32);
  want_dim(ss, "s", 3);
  const int64_t e = ss.shape[0], n = ss.shape[1], k = ss.shape[2] * 32;
  if (ww.numel() != e * n * (k / 128)) throw std::runtime_error("words must hold E*N*K/128 ints");
  check(hkmoe_mx_pack_weight_scales(ss.ptr, e, n, k, gate_up, ww.ptr, current_stream()));
}

void dispatch_mx_gather_scales(py::object s, py::object gather, int32_t gather_div, py::object offsets,
                               py::object mtile_offsets, int64_t rows, py::object words) {
  auto ss = as_tensor(s, "s"), g = as_tensor_opt(gather, "gather"), o = as_tensor(offsets, "offsets"),
       mo = as_tensor(mtile_offsets, "mtile_offsets"), ww = as_tensor(words, "words");
  want_dtype(ss, "s", kU8);
  want_dtype(g, "gather", kI32);
  want_dtype(ww, "words", kI32);
  want_dim(ss, "s", 2);
  const int64_t x_rows = ss.shape[0], k = ss.shape[1] * 32, e = o.numel() - 1;
  if (mo.numel() != e + 1) throw std::runtime_error("offsets and mtile_offsets must hold E+1 values");
  if (g.ptr && g.numel() != rows) throw std::runtime_error("gather must hold one index per row");
  if (ww.numel() != (k / 128) * mx_ws(rows, e)) throw std::runtime_error("words must be [K/128, ws]");
  check(hkmoe_mx_gather_scales(ss.ptr, x_rows, static_cast<int32_t>(k), static_cast<const int32_t*>(g.ptr),
                               gather_div, static_cast<const int32_t*>(o.ptr),
                               static_cast<const int32_t*>(mo.ptr), static_cast<int32_t>(e), rows, ww.ptr,
                               current_stream()));
}

void dispatch_grouped_gemm1_mx(py::object x_q, py::object x_words, py::object gather, int32_t gather_div,
                               py::object w13, py::object w13_words, py::object offsets,
                               py::object mtile_offsets, py::object h, py::object h_words,
                               py::object tile_counters, bool packed, py::object mtile_list) {
  auto x = as_tensor(x_q, "x"), xw = as_tensor(x_words, "x_words"), gth = as_tensor_opt(gather, "gather"),
       w = as_tensor(w13, "w13"), ww = as_tensor(w13_words, "w13_words"), o = as_tensor(offsets, "offsets"),
       mo = as_tensor(mtile_offsets, "mtile_offsets"), hh = as_tensor(h, "h"),
       hw = as_tensor_opt(h_words, "h_words"), tc = as_tensor_opt(tile_counters, "tile_counters"),
       ml = as_tensor_opt(mtile_list, "mtile_list");
  want_dtype(x, "x", kF8);
  want_dtype(w, "w13", kF8);
  want_dtype(xw, "x_words", kI32);
  want_dtype(ww, "w13_words", kI32);
  want_dtype(hw, "h_words", kI32);
  want_dtype(gth, "gather", kI32);
  want_dtype(tc, "tile_counters", kI32);
  want_dtype(ml, "mtile_list", kI32);
  want_dim(x, "x", 2);
  want_dim(w, "w13", 3);
  want_dim(hh, "h", 2);
  if (tc.ptr && tc.numel() < 8) throw std::runtime_error("tile_counters must hold 8 ints");
  const int64_t x_rows = x.shape[0], hidden = x.shape[1], e = w.shape[0], inter = w.shape[1] / 2;
  const int64_t rows = hh.shape[0];
  if (w.shape[2] != hidden || w.shape[1] % 2) throw std::runtime_error("w13 must be [E, 2I, H]");
  if (hh.shape[1] != inter) throw std::runtime_error("h must be [rows, I]");
  if (gth.ptr && gth.numel() != rows) throw std::runtime_error("gather must hold one index per row");
  if (ml.ptr && ml.numel() < mtile_list_ints(rows, e)) throw std::runtime_error("mtile_list too small");
  if (o.numel() != e + 1 || mo.numel() != e + 1) throw std::runtime_error("offsets must hold E+1 values");
  if (xw.numel() != (hidden / 128) * mx_ws(rows, e)) throw std::runtime_error("x_words must be [H/128, ws]");
  if (ww.numel() != e * 2 * inter * (hidden / 128)) throw std::runtime_error("w13_words must hold E*2I*H/128 ints");
  int fmt;
  if (hh.dtype == kBf16) fmt = HKMOE_BF16;
  else if (hh.dtype == kF8) fmt = HKMOE_E4M3;
  else throw std::runtime_error("h: expected bfloat16 or float8_e4m3fn");
  if (fmt == HKMOE_E4M3 && ((rows > 0 && !hw.ptr) || hw.numel() != (inter / 128) * mx_ws(rows, e)))
    throw std::runtime_error("e4m3 output needs h_words [I/128, ws]");
  check(hkmoe_grouped_gemm1_mx(x.ptr, xw.ptr, static_cast<const int32_t*>(gth.ptr), gather_div, x_rows, w.ptr,
                               ww.ptr, static_cast<const int32_t*>(o.ptr), static_cast<const int32_t*>(mo.ptr),
                               static_cast<const int32_t*>(ml.ptr), rows, static_cast<int32_t>(e),
                               static_cast<int32_t>(hidden), static_cast<int32_t>(inter),
                               packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, fmt, hh.ptr, hw.ptr,
                               static_cast<int32_t*>(tc.ptr), current_stream()));
}

void dispatch_grouped_gemm2_mx(py::object hq, py::object hq_words, py::object w2, py::object w2_words,
                               py::object offsets, py::object mtile_offsets, py::object y,
                               py::object tile_counters, bool packed, py::object mtile_list) {
  auto q = as_tensor(hq, "hq"), qw = as_tensor(hq_words, "hq_words"), w = as_tensor(w2, "w2"),
       ww = as_tensor(w2_words, "w2_words"), o = as_tensor(offsets, "offsets"),
       mo = as_tensor(mtile_offsets, "mtile_offsets"), yy = as_tensor(y, "y"),
       tc = as_tensor_opt(tile_counters, "tile_counters"), ml = as_tensor_opt(mtile_list, "mtile_list");
  want_dtype(q, "hq", kF8);
  want_dtype(w, "w2", kF8);
  want_dtype(qw, "hq_words", kI32);
  want_dtype(ww, "w2_words", kI32);
  want_dtype(yy, "y", kBf16);
  want_dtype(tc, "tile_counters", kI32);
  want_dtype(ml, "mtile_list", kI32);
  want_dim(q, "hq", 2);
  want_dim(w, "w2", 3);
  if (tc.ptr && tc.numel() < 8) throw std::runtime_error("tile_counters must hold 8 ints");
  const int64_t rows = q.shape[0], inter = q.shape[1], e = w.shape[0], hidden = w.shape[1];
  if (w.shape[2] != inter) throw std::runtime_error("w2 must be [E, H, I]");
  if (yy.numel() != rows * hidden) throw std::runtime_error("y must be [rows, H]");
  if (o.numel() != e + 1 || mo.numel() != e + 1) throw std::runtime_error("offsets must hold E+1 values");
  if (ml.ptr && ml.numel() < mtile_list_ints(rows, e)) throw std::runtime_error("mtile_list too small");
  if (qw.numel() != (inter / 128) * mx_ws(rows, e)) throw std::runtime_error("hq_words must be [I/128, ws]");
  if (ww.numel() != e * hidden * (inter / 128)) throw std::runtime_error("w2_words must hold E*H*I/128 ints");
  check(hkmoe_grouped_gemm2_mx(q.ptr, qw.ptr, w.ptr, ww.ptr, static_cast<const int32_t*>(o.ptr),
                               static_cast<const int32_t*>(mo.ptr), static_cast<const int32_t*>(ml.ptr), rows,
                               static_cast<int32_t>(e), static_cast<int32_t>(hidden),
                               static_cast<int32_t>(inter), packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, yy.ptr,
                               static_cast<int32_t*>(tc.ptr), current_stream()));
}

void dispatch_moe_mx(py::object x_q, py::object x_e8m0, py::object logits, py::object w13, py::object w13_words,
                     py::object w2, py::object w2_words, int32_t top_k, py::object out, py::object workspace,
                     bool packed) {
  auto x = as_tensor(x_q, "x_q"), xe = as_tensor(x_e8m0, "x_e8m0"), l = as_tensor(logits, "logits"),
       a = as_tensor(w13, "w13"), aw = as_tensor(w13_words, "w13_words"), b = as_tensor(w2, "w2"),
       bw = as_tensor(w2_words, "w2_words"), o = as_tensor(out, "out"), ws = as_tensor(workspace, "workspace");
  want_dtype(x, "x_q", kF8);
  want_dtype(a, "w13", kF8);
  want_dtype(b, "w2", kF8);
  want_dtype(xe, "x_e8m0", kU8);
  want_dtype(aw, "w13_words", kI32);
  want_dtype(bw, "w2_words", kI32);
  want_dtype(l, "logits", kF32);
  want_dtype(o, "out", kBf16);
  want_dim(x, "x_q", 2);
  want_dim(l, "logits", 2);
  want_dim(a, "w13", 3);
  want_dim(b, "w2", 3);
  const int64_t t = x.shape[0], hidden = x.shape[1], e = a.shape[0], inter = a.shape[1] / 2;
  if (l.shape[0] != t || l.shape[1] != e) throw std::runtime_error("logits must be [T, E]");
  if (a.shape[2] != hidden || b.shape[0] != e || b.shape[1] != hidden || b.shape[2] != inter)
    throw std::runtime_error("w13 must be [E, 2I, H] and w2 [E, H, I]");
  if (o.numel() != t * hidden) throw std::runtime_error("out must be [T, H]");
  if (xe.numel() != t * (hidden / 32)) throw std::runtime_error("x_e8m0 must be [T, H/32]");
  if (aw.numel() != e * 2 * inter * (hidden / 128) || bw.numel() != e * hidden * (inter / 128))
    throw std::runtime_error("weight words: w13_words E*2I*H/128, w2_words E*H*I/128 ints");
  const size_t bytes = static_cast<size_t>(ws.numel()) * (ws.dtype == kF32 || ws.dtype == kI32 ? 4 : 1);
  check(hkmoe_moe_forward_mx(x.ptr, xe.ptr, static_cast<const float*>(l.ptr), a.ptr, aw.ptr, b.ptr, bw.ptr, t,
                             static_cast<int32_t>(e), top_k, static_cast<int32_t>(hidden),
                             static_cast<int32_t>(inter), packed ? HKMOE_W_PACKED : HKMOE_W_ROWS, o.ptr, ws.ptr,
                             bytes, current_stream()));
}

}  // namespace

PYBIND11_MODULE(tk_kernel, m) {
  m.doc() = "gfx950 FP8 MoE grouped-GEMM path (dispatch_* entry points over the hkmoe C ABI)";
  m.def("dispatch_micro", &dispatch_micro, "C = A . B^T (e4m3 in, fp32/bf16 out, unit scales)");
  m.def("dispatch_gemm_fp8", &dispatch_gemm, "C = (sa*sb) A . B^T, per-tensor scales",
        py::arg("A"), py::arg("B"), py::arg("C"), py::arg("scale_a") = py::none(),
        py::arg("scale_b") = py::none());
  m.def("dispatch_route_topk", &dispatch_route_topk);
  m.def("dispatch_expert_offsets", &dispatch_expert_offsets, py::arg("block_counts"), py::arg("num_tokens"),
        py::arg("counts"), py::arg("offsets"), py::arg("block_base"), py::arg("mtile_offsets"),
        py::arg("amax") = py::none(), py::arg("tile_counters") = py::none(),
        py::arg("mtile_list") = py::none(), py::arg("narrow_max") = 0, py::arg("narrow_info") = py::none());
  m.def("dispatch_scatter", &dispatch_scatter);
  m.def("dispatch_grouped_gemm1", &dispatch_grouped_gemm1, py::arg("x_q"), py::arg("x_scale"), py::arg("gather"),
        py::arg("gather_div"), py::arg("w13"), py::arg("w13_scale"), py::arg("offsets"),
        py::arg("mtile_offsets"), py::arg("h"), py::arg("h_aux") = py::none(),
        py::arg("tile_counters") = py::none(), py::arg("packed") = false, py::arg("mtile_list") = py::none(),
        py::arg("narrow_info") = py::none(), py::arg("part") = 0, py::arg("grid") = 0);
  m.def("dispatch_requant", &dispatch_requant);
  m.def("dispatch_requant_quotient_check", &dispatch_requant_quotient_check);
  m.def("dispatch_grouped_gemm2", &dispatch_grouped_gemm2, py::arg("hq"), py::arg("hs"), py::arg("w2"),
        py::arg("w2_scale"), py::arg("offsets"), py::arg("mtile_offsets"), py::arg("y"),
        py::arg("tile_counters") = py::none(), py::arg("packed") = false, py::arg("mtile_list") = py::none(),
        py::arg("narrow_info") = py::none(), py::arg("part") = 0, py::arg("grid") = 0);
  m.def("dispatch_combine", &dispatch_combine);
  m.def("dispatch_moe", &dispatch_moe, py::arg("x_q"), py::arg("x_scale"), py::arg("logits"), py::arg("w13"),
        py::arg("w13_scale"), py::arg("w2"), py::arg("w2_scale"), py::arg("top_k"), py::arg("out"),
        py::arg("workspace"), py::arg("packed") = false);
  m.def("dispatch_pack_weights", &dispatch_pack_weights, py::arg("w"), py::arg("packed"), py::arg("gate_up"));
  m.def("dispatch_quant_group", &dispatch_quant_group);
  m.def("dispatch_quant_block", &dispatch_quant_block);
  m.def("dispatch_quant_tensor", &dispatch_quant_tensor);
  m.def("dispatch_quant_mx", &dispatch_quant_mx, "x fp32 [R,C] -> q e4m3 [R,C], e8m0 s uint8 [R,C/32]");
  m.def("dispatch_mx_pack_scales", &dispatch_mx_pack_scales, py::arg("s"), py::arg("cols"), py::arg("packed"));
  m.def("mx_words_per_step", &mx_ws, "words per K step of the tile-aligned MX exponent layouts");
  m.def("dispatch_mx_pack_weight_scales", &dispatch_mx_pack_weight_scales, py::arg("s"), py::arg("words"),
        py::arg("gate_up"));
  m.def("dispatch_mx_gather_scales", &dispatch_mx_gather_scales, py::arg("s"), py::arg("gather"),
        py::arg("gather_div"), py::arg("offsets"), py::arg("mtile_offsets"), py::arg("rows"), py::arg("words"));
  m.def("dispatch_grouped_gemm1_mx", &dispatch_grouped_gemm1_mx, py::arg("x_q"), py::arg("x_words"),
        py::arg("gather"), py::arg("gather_div"), py::arg("w13"), py::arg("w13_words"), py::arg("offsets"),
        py::arg("mtile_offsets"), py::arg("h"), py::arg("h_words") = py::none(),
        py::arg("tile_counters") = py::none(), py::arg("packed") = false, py::arg("mtile_list") = py::none());
  m.def("dispatch_grouped_gemm2_mx", &dispatch_grouped_gemm2_mx, py::arg("hq"), py::arg("hq_words"),
        py::arg("w2"), py::arg("w2_words"), py::arg("offsets"), py::arg("mtile_offsets"), py::arg("y"),
        py::arg("tile_counters") = py::none(), py::arg("packed") = false, py::arg("mtile_list") = py::none());
  m.def("dispatch_moe_mx", &dispatch_moe_mx, py::arg("x_q"), py::arg("x_e8m0"), py::arg("logits"),
        py::arg("w13"), py::arg("w13_words"), py::arg("w2"), py::arg("w2_words"), py::arg("top_k"),
        py::arg("out"), py::arg("workspace"), py::arg("packed") = true);
  m.def("dispatch_gemm_mx", &dispatch_gemm_mx, "C = A . B^T with 1x32 e8m0 scales (packed words)",
        py::arg("A"), py::arg("scale_a"), py::arg("B"), py::arg("scale_b"), py::arg("C"));
  m.def("moe_workspace_size", &moe_workspace_size);
  m.def("set_narrow", [](int cus, int max_rows, int wide_share) { check(hkmoe_set_narrow(cus, max_rows, wide_share)); },
        "narrow path of dispatch_moe: workgroups (0 = off), largest expert it takes, wide-GEMM CU share",
        py::arg("cus"), py::arg("max_rows") = 64, py::arg("wide_share") = 0);
  m.def("get_narrow", []() {
    int32_t c = 0, r = 0, w = 0;
    check(hkmoe_get_narrow(&c, &r, &w));
    return py::make_tuple(c, r, w);
  });
  m.def("kernel_timing", [](int calls) { check(hkmoe_kernel_timing(calls)); },
        "time the kernels of the next layer calls (per-dispatch events, a ring of `calls` sets); 0 = off",
        py::arg("calls"));
  m.def("kernel_timing_read", [](int set) {
    std::vector<float> b(HKMOE_TIMING_ROLES), e(HKMOE_TIMING_ROLES);
    check(hkmoe_kernel_timing_read(set, b.data(), e.data(), HKMOE_TIMING_ROLES));
    py::list out;
    for (int r = 0; r < HKMOE_TIMING_ROLES; ++r) out.append(py::make_tuple(b[r], e[r]));
    return out;
  }, "(start, end) ms of each role's kernel from the start of the call's first kernel ((-1, -1): not launched)",
        py::arg("set"));
  m.attr("TIMING_ROLES") = py::make_tuple("route_topk", "expert_block_scan", "expert_offsets", "scatter",
                                          "mx_gather_words", "grouped_gemm1", "narrow_gemm1", "grouped_gemm1_join",
                                          "requant", "grouped_gemm2", "narrow_gemm2", "combine");
  m.def("set_dense_mfma", [](int shape) { check(hkmoe_set_dense_mfma(shape)); },
        "MFMA shape (16 or 32) of the 128x128-tile dense GEMM kernel", py::arg("shape"));
  m.def("get_dense_mfma", []() { return hkmoe_get_dense_mfma(); });
  m.def("route_blocks", [](int64_t t) { return hkmoe_route_blocks(t); });
  m.def("mtile_list_ints", &mtile_list_ints, "ints of an M-tile list for `rows` expert rows over E experts");
  m.def("version", []() { return hkmoe_version(); });
  m.attr("SCALE_TENSOR") = static_cast<int>(HKMOE_SCALE_TENSOR);
  m.attr("SCALE_BLOCK") = static_cast<int>(HKMOE_SCALE_BLOCK);
  m.attr("SCALE_MX") = static_cast<int>(HKMOE_SCALE_MX);
}
