// Eager host path of the W8A8 linear and the fused quantizers: the same C-ABI launches as
// the ctypes path of int8_linear/kernel.py and int8_linear/fused_quant.py, with the argument
// checks, the configuration lookup, the output allocation and the stream lookup done in C++
// rather than in Python.  Host code only (built by g++ against torch's headers); the kernels
// stay behind include/int8_linear_amd.h, and no torch type crosses that boundary.
//
// Every function returns None instead of launching when anything about its arguments is
// not the plain case (a dtype, device, layout or size the C path would reject or that the
// Python layer first copies), and the Python wrapper then takes its own path, which raises
// the reference's exception for the same input (AshrithaG/int8-linear int8_linear/kernel.py
// 221-242, int8_linear/fused_quant.py:89-124).  So this module changes the host cost of a
// call, never its result or its errors.
//
// Configuration choice follows kernel.choose_config (reference kernel.py:137-160): per
// device, the tuned table's largest M bucket at or below M for "KxN", else the library's
// default rule.  Python hands each device's table over once (set_table) before the first
// fast call on that device.

#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <map>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/int8_linear_amd.h"

namespace {

namespace py = pybind11;

int32_t float_code(at::ScalarType t) {
  switch (t) {
    case at::kBFloat16: return I8L_BF16;
    case at::kHalf: return I8L_F16;
    case at::kFloat: return I8L_F32;
    default: return -1;
  }
}

int32_t act_code(at::ScalarType t) {
  return t == at::kBFloat16 ? I8L_BF16 : t == at::kHalf ? I8L_F16 : -1;
}

void* stream_of(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Tuned configurations of one device: "KxN" -> M bucket -> config.
using ShapeTable = std::map<int64_t, i8l_config>;
struct DeviceTable {
  std::unordered_map<uint64_t, ShapeTable> shapes;
};
std::unordered_map<int, DeviceTable> g_tables;

uint64_t kn_key(int64_t k, int64_t n) { return ((uint64_t)k << 32) ^ (uint64_t)n; }

// rows: (k, n, m_bucket, bm, bn, bk, warps, stages, group_m)
void set_table(int device, const std::vector<std::vector<int64_t>>& rows) {
  DeviceTable t;
  for (const auto& r : rows) {
    TORCH_CHECK(r.size() == 9, "a tuned row has 9 fields");
    i8l_config c{(int32_t)r[3], (int32_t)r[4], (int32_t)r[5], (int32_t)r[6],
                 (int32_t)r[7], (int32_t)r[8]};
    t.shapes[kn_key(r[0], r[1])][r[2]] = c;
  }
  g_tables[device] = std::move(t);
}

bool has_table(int device) { return g_tables.count(device) != 0; }

// false when the device's table has not been handed over yet
bool choose(int device, int64_t m, int64_t n, int64_t k, i8l_config* c) {
  auto dt = g_tables.find(device);
  if (dt == g_tables.end()) return false;
  auto st = dt->second.shapes.find(kn_key(k, n));
  if (st != dt->second.shapes.end()) {
    auto it = st->second.upper_bound(m);  // first bucket above M
    if (it != st->second.begin()) {
      *c = std::prev(it)->second;
      return true;
    }
  }
  return i8l_default_config(m, n, k, c) == I8L_OK;
}

// The configuration the fast path launches (bm, bn, bk, warps, stages, group_m),
// or None before the device's table is handed over.
py::object config_for(int device, int64_t m, int64_t n, int64_t k) {
  i8l_config c;
  if (!choose(device, m, n, k, &c)) return py::none();
  return py::make_tuple(c.bm, c.bn, c.bk, c.warps, c.stages, c.group_m);
}

// Launches made through this module (every entry point), for tests that check it was used.
int64_t g_launches = 0;

bool plain_vector(const at::Tensor& t, at::ScalarType dt, const at::Device& dev) {
  return t.scalar_type() == dt && t.device() == dev && t.is_contiguous();
}

// w8a8_mm(a_q, b_q, scale_a, scale_b, out_dtype, bias) with the configuration chosen here.
py::object mm(const at::Tensor& a, const at::Tensor& b, const at::Tensor& sa,
              const at::Tensor& sb, at::ScalarType out_dtype,
              const c10::optional<at::Tensor>& bias) {
  if (a.scalar_type() != at::kChar || b.scalar_type() != at::kChar || a.dim() != 2 ||
      b.dim() != 2 || !a.is_cuda())
    return py::none();
  const at::Device dev = a.device();
  const int64_t m = a.size(0), k = a.size(1), n = b.size(1);
  if (b.size(0) != k || b.device() != dev) return py::none();
  i8l_config c;
  if (!choose(dev.index(), m, n, k, &c) || c.bn <= 0 || c.bk <= 0 || n % c.bn || k % c.bk)
    return py::none();
  if (!plain_vector(sa, at::kFloat, dev) || !plain_vector(sb, at::kFloat, dev)) return py::none();
  if ((sa.numel() != 1 && sa.numel() != m) || (sb.numel() != 1 && sb.numel() != n))
    return py::none();
  const int32_t out_code = float_code(out_dtype);
  if (out_code < 0) return py::none();
  int32_t bias_code = I8L_DTYPE_NONE;
  const void* bias_ptr = nullptr;
  if (bias.has_value()) {
    const at::Tensor& bt = *bias;
    bias_code = float_code(bt.scalar_type());
    if (bias_code < 0 || bt.dim() != 1 || bt.size(0) != n || bt.device() != dev ||
        !bt.is_contiguous())
      return py::none();
    bias_ptr = bt.data_ptr();
  }
  at::Tensor out = at::empty({m, n}, a.options().dtype(out_dtype));
  // a split of K takes its int32 partial planes from the caching allocator (stream-ordered,
  // and from the graph's pool under capture)
  const int64_t ws_bytes = i8l_w8a8_mm_workspace_bytes(m, n, k, &c);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({ws_bytes}, a.options().dtype(at::kByte));
  const int st = i8l_w8a8_mm_ws(
      (const int8_t*)a.data_ptr(), a.stride(0), a.stride(1), (const int8_t*)b.data_ptr(),
      b.stride(0), b.stride(1), (const float*)sa.data_ptr(), sa.numel(),
      (const float*)sb.data_ptr(), sb.numel(), bias_ptr, bias_code, out.data_ptr(),
      out.stride(0), out_code, m, n, k, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, &c,
      stream_of(a));
  if (st != I8L_OK) return py::none();
  ++g_launches;
  return py::cast(out);
}

py::object add_rmsnorm_quant(const at::Tensor& x, const c10::optional<at::Tensor>& residual,
                             const at::Tensor& w, double eps, bool precise_div) {
  if (x.dim() != 2 || !x.is_cuda() || !x.is_contiguous()) return py::none();
  const int32_t act = act_code(x.scalar_type()), wcode = act_code(w.scalar_type());
  const int64_t M = x.size(0), H = x.size(1);
  if (act < 0 || wcode < 0 || w.numel() != H || w.device() != x.device() || !w.is_contiguous())
    return py::none();
  at::Tensor rout;
  const void* rptr = nullptr;
  if (residual.has_value()) {
    const at::Tensor& r = *residual;
    if (!r.is_contiguous() || r.sizes() != x.sizes() || r.scalar_type() != x.scalar_type() ||
        r.device() != x.device())
      return py::none();
    rptr = r.data_ptr();
    rout = at::empty_like(x);
  }
  at::Tensor q = at::empty({M, H}, x.options().dtype(at::kChar));
  at::Tensor s = at::empty({M, 1}, x.options().dtype(at::kFloat));
  if (M) {
    const int st = i8l_add_rmsnorm_quant(x.data_ptr(), rptr, w.data_ptr(), (float)eps,
                                         (int8_t*)q.data_ptr(), (float*)s.data_ptr(),
                                         rout.defined() ? rout.data_ptr() : nullptr, M, H, act,
                                         wcode, precise_div ? 1 : 0, stream_of(x));
    if (st != I8L_OK) return py::none();
    ++g_launches;
  }
  return py::make_tuple(q, s, rout.defined() ? py::cast(rout) : py::none());
}

py::object silu_mul_quant(const at::Tensor& gu, bool precise_div, bool round_silu) {
  if (gu.dim() != 2 || !gu.is_cuda() || !gu.is_contiguous()) return py::none();
  const int32_t act = act_code(gu.scalar_type());
  if (act < 0) return py::none();
  const int64_t M = gu.size(0), I = gu.size(1) / 2;
  at::Tensor q = at::empty({M, I}, gu.options().dtype(at::kChar));
  at::Tensor s = at::empty({M, 1}, gu.options().dtype(at::kFloat));
  if (M && I) {
    const int st = i8l_silu_mul_quant(gu.data_ptr(), (int8_t*)q.data_ptr(), (float*)s.data_ptr(),
                                      M, I, act, round_silu ? 1 : 0, precise_div ? 1 : 0,
                                      stream_of(gu));
    if (st != I8L_OK) return py::none();
    ++g_launches;
  }
  return py::make_tuple(q, s);
}

py::object quant_per_token(const at::Tensor& x, bool precise_div) {
  if (x.dim() != 2 || !x.is_cuda()) return py::none();
  const int64_t M = x.size(0), H = x.size(1);
  if (x.stride(1) != 1 && H > 1) return py::none();
  const int32_t act = act_code(x.scalar_type());
  if (act < 0) return py::none();
  at::Tensor q = at::empty({M, H}, x.options().dtype(at::kChar));
  at::Tensor s = at::empty({M, 1}, x.options().dtype(at::kFloat));
  if (M && H) {
    const int64_t ldx = M > 1 ? x.stride(0) : H;
    const int st = i8l_quant_per_token(x.data_ptr(), ldx, (int8_t*)q.data_ptr(),
                                       (float*)s.data_ptr(), M, H, act, precise_div ? 1 : 0,
                                       stream_of(x));
    if (st != I8L_OK) return py::none();
    ++g_launches;
  }
  return py::make_tuple(q, s);
}

}  // namespace

PYBIND11_MODULE(_i8l_fast, m) {
  m.doc() = "C++ eager host path over the int8_linear_amd C ABI";
  m.def("set_table", &set_table, "hand over one device's tuned configurations");
  m.def("has_table", &has_table);
  m.def("config_for", &config_for);
  m.def("launches", [] { return g_launches; });
  m.def("mm", &mm, py::arg("a_q"), py::arg("b_q"), py::arg("scale_a"), py::arg("scale_b"),
        py::arg("out_dtype"), py::arg("bias"));
  m.def("add_rmsnorm_quant", &add_rmsnorm_quant);
  m.def("silu_mul_quant", &silu_mul_quant);
  m.def("quant_per_token", &quant_per_token);
}
