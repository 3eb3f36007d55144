// Request-level lifecycle of libxrmm: plan / prepare / run / read_outputs /
// info / close for the three MatMulNBits-family operators and for
// com.microsoft.QMoE (1030), GatherBlockQuantized (1031) and MatMulBnb4 (1026).
//
// Behaviour follows xrgpu::operators::extended:
//  * plan():   contract validation (kernels/_shared/extended/contracts.cpp:14,
//              rows contract_data.h:659-663,718-751,821-827), args-over-attrs
//              merging (planner.cpp:67-85), attribute defaults, checks and
//              output shapes of the complex planner (complex_plan.cpp:117-129),
//              requested-output checks (planner.cpp:86-93);
//  * prepare(): input byte-count and memory-limit checks (planner.cpp:32-49),
//              then one device arena holding every input and output;
//  * run():    launch on the operator's own stream and wait with a time-out;
//              any failure poisons the operator (vulkan.cpp:105,115);
//  * read_outputs(): device-to-host copy plus storage-dtype conversion
//              (planner.cpp:51-66);
//  * info():   JSON like vulkan.cpp:123 (execution_ms, gpu_ms, ...).
// Error classes: XRMM_EINVAL where the reference throws std::invalid_argument,
// XRMM_EDEVICE where it throws std::runtime_error.
//
// Deliberate differences, all stricter: B/scales/zero-point/bias/normScale
// shapes are checked on the host (the reference detects a malformed B only on
// the GPU), A's last dimension must equal K, and Nq/Nkv must be positive.
// Extension ports: packed uint8 zeroPointsT; q/k/vZeroPointsT for Qkv and
// gate/upZeroPointsT for Mlp.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/xrmm.h"
#include "xrmm_internal.h"
#include "xrmm_moe.h"
#include "xrmm_quant.h"

namespace {

// Exceptions of the two classes, converted to status codes at the ABI edge.
struct Invalid : std::invalid_argument {
  using std::invalid_argument::invalid_argument;
};
struct Device : std::runtime_error {
  using std::runtime_error::runtime_error;
};

uint32_t dtype_bytes(int32_t d) {
  switch (d) {
    case XRMM_F32: case XRMM_I32: case XRMM_U32: return 4;
    case XRMM_F16: case XRMM_I16: return 2;
    case XRMM_I8: case XRMM_U8: case XRMM_BOOL: return 1;
    case XRMM_I64: return 8;
    default: throw Invalid("Unsupported dtype");
  }
}

bool floating(int32_t d) { return d == XRMM_F32 || d == XRMM_F16; }

const char* dtype_name(int32_t d) {
  static const char* names[] = {"float32", "float16", "int32", "uint32", "int16", "int8", "uint8", "int64", "bool", "unspecified"};
  return d >= 0 && d <= XRMM_UNSPECIFIED ? names[d] : "invalid";
}

struct Tensor {
  std::string name;
  int32_t dtype = XRMM_UNSPECIFIED;
  int32_t storage = XRMM_UNSPECIFIED;  // resolved: never UNSPECIFIED for a present tensor
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  uint64_t nbytes = 0;
};

uint64_t numel(const std::vector<int64_t>& s) {
  uint64_t n = 1;
  for (int64_t d : s) {
    if (d < 0) throw Invalid("Negative tensor dimension");
    if (d && n > (uint64_t(1) << 62) / uint64_t(d)) throw Invalid("Tensor element count overflow");
    n *= uint64_t(d);
  }
  return n;
}

// One contract row: port name, type variable, dtype mask, rank (-1: any),
// optional. Masks use bit (1 << dtype).
struct Port {
  const char* name;
  const char* var;
  uint32_t mask;
  int rank;
  bool optional;
};

constexpr uint32_t kT1 = (1u << XRMM_F32) | (1u << XRMM_F16);
constexpr uint32_t kU8 = 1u << XRMM_U8;
constexpr uint32_t kT3 = kT1 | kU8;  // float zero points (reference) or packed uint8 (extension)
constexpr uint32_t kF32 = 1u << XRMM_F32;
// int64 indices (the reference contract) and int32 / uint32 (read as int32 by controlIndex)
// GatherBlockQuantized indices: Tind = int64 in the reference contract
// (contract_data.h:660); int32 / uint32 indices are taken only by the
// zero-copy entry point.
constexpr uint32_t kIdx = 1u << XRMM_I64;
// operators outside the MatMulNBits family (xrmm::Op covers that family)
constexpr int OP_BNB4 = 10, OP_QMOE = 11, OP_GBQ = 12;

struct OpContract {
  const char* operation;
  int op;  // xrmm::Op
  std::vector<Port> inputs;
  std::vector<Port> outputs;
};

const std::vector<OpContract>& contracts() {
  static const std::vector<OpContract> c = {
      {"com.microsoft.MatMulNBits", xrmm::OP_MATMUL,
       {{"aT", "T1", kT1, -1, false}, {"bT", "", kU8, 3, false}, {"scalesT", "T1", kT1, 2, false},
        {"zeroPointsT", "T3", kT3, 2, true}, {"biasT", "T1", kT1, 1, true}},
       {{"yT", "T1", kT1, -1, false}}},
      {"com.microsoft.MatMulNBitsMlp", xrmm::OP_MLP,
       {{"aT", "T1", kT1, -1, false}, {"skipT", "T1", kT1, -1, true}, {"normScaleT", "T1", kT1, 1, true},
        {"gateBT", "", kU8, 3, false}, {"gateScalesT", "T1", kT1, 2, false}, {"gateBiasT", "T1", kT1, 1, true},
        {"upBT", "", kU8, 3, false}, {"upScalesT", "T1", kT1, 2, false}, {"upBiasT", "T1", kT1, 1, true},
        {"gateZeroPointsT", "T3", kT3, 2, true}, {"upZeroPointsT", "T3", kT3, 2, true}},
       {{"yT", "T1", kT1, -1, false}, {"residualT", "T1", kT1, -1, true}}},
      {"com.microsoft.MatMulNBitsQkv", xrmm::OP_QKV,
       {{"aT", "T1", kT1, -1, false}, {"skipT", "T1", kT1, -1, true}, {"normScaleT", "T1", kT1, 1, false},
        {"qBT", "T2", kU8, 3, false}, {"qScalesT", "T1", kT1, 2, false}, {"kBT", "T2", kU8, 3, false},
        {"kScalesT", "T1", kT1, 2, false}, {"vBT", "T2", kU8, 3, false}, {"vScalesT", "T1", kT1, 2, false},
        {"qZeroPointsT", "T3", kT3, 2, true}, {"kZeroPointsT", "T3", kT3, 2, true}, {"vZeroPointsT", "T3", kT3, 2, true}},
       {{"qT", "T1", kT1, -1, false}, {"kT", "T1", kT1, -1, false}, {"vT", "T1", kT1, -1, false},
        {"residualT", "T1", kT1, -1, true}}},
      {"com.microsoft.MatMulBnb4", OP_BNB4,
       {{"aT", "T1", kT1, 2, false}, {"bT", "T2", kU8, 1, false}, {"absmaxT", "T1", kT1, 1, false}},
       {{"yT", "T1", kT1, 2, false}}},
      {"com.microsoft.QMoE", OP_QMOE,
       {{"inputT", "T", kF32, -1, false}, {"routerT", "T", kF32, 2, false}, {"fc1T", "T1", kU8, 3, false},
        {"fc1ScalesT", "T2", kF32, -1, false}, {"fc2T", "T1", kU8, 3, false}, {"fc2ScalesT", "T2", kF32, -1, false}},
       {{"outputT", "T", kF32, -1, false}}},
      {"com.microsoft.GatherBlockQuantized", OP_GBQ,
       {{"dataT", "T1", kU8, 2, false}, {"indicesT", "Tind", kIdx, 1, false}, {"scalesT", "T2", kF32, 2, false},
        {"zeroPointsT", "T1", kU8, 2, true}},
       {{"outputT", "T2", kF32, 2, false}}},
  };
  return c;
}

struct Attr {
  int kind;
  int64_t i;
  double f;
  std::string s;
};
using Attrs = std::map<std::string, Attr>;

Tensor from_c(const xrmm_tensor& t, bool payload) {
  Tensor r;
  if (!t.name || !*t.name) throw Invalid("Duplicate or unnamed extended input");
  r.name = t.name;
  r.dtype = t.dtype;
  if (r.dtype == XRMM_UNSPECIFIED) throw Invalid("Missing logical dtype");
  if (r.dtype < 0 || r.dtype > XRMM_BOOL) throw Invalid("Unsupported dtype: " + r.name);
  r.storage = t.storage_dtype == XRMM_UNSPECIFIED ? t.dtype : t.storage_dtype;
  if (r.storage < 0 || r.storage > XRMM_BOOL) throw Invalid("Unsupported storage dtype: " + r.name);
  if (floating(r.dtype) != floating(r.storage)) throw Invalid("Logical/storage float versus integer types differ");
  if (t.rank < 0 || t.rank > XRMM_MAX_RANK) throw Invalid("Rank outside the supported range: " + r.name);
  r.shape.assign(t.shape, t.shape + t.rank);
  numel(r.shape);
  if (payload) {
    r.data = static_cast<const uint8_t*>(t.data);
    r.nbytes = t.nbytes;
  }
  return r;
}

Attrs merged_attrs(const xrmm_request& q) {
  // args take precedence over attrs key by key (planner.cpp:67-85)
  Attrs a;
  auto add = [&](const xrmm_attr* v, int32_t n) {
    if (n < 0 || (n > 0 && !v)) throw Invalid("Invalid attribute list");
    for (int32_t i = 0; i < n; ++i) {
      if (!v[i].key) throw Invalid("Unnamed attribute");
      if (v[i].kind < XRMM_ATTR_INT || v[i].kind > XRMM_ATTR_STRING) throw Invalid(std::string("Unsupported attribute kind: ") + v[i].key);
      a[v[i].key] = Attr{v[i].kind, v[i].i, v[i].f, v[i].kind == XRMM_ATTR_STRING && v[i].s ? v[i].s : ""};
    }
  };
  add(q.attrs, q.n_attrs);
  add(q.args, q.n_args);
  return a;
}

// numeric_integer / numeric_attr / attr_s of kernels/_shared/extended/framework.h:30-35
int64_t attr_int(const Attrs& a, const std::string& n, int64_t fallback) {
  auto it = a.find(n);
  if (it == a.end()) return fallback;
  if (it->second.kind == XRMM_ATTR_INT) return it->second.i;
  if (it->second.kind == XRMM_ATTR_FLOAT) {
    const double v = it->second.f;
    if (!std::isfinite(v) || std::trunc(v) != v || std::fabs(v) >= 9.2e18) throw Invalid("Integer attribute required: " + n);
    return int64_t(v);
  }
  return fallback;
}

double attr_num(const Attrs& a, const std::string& n, double fallback) {
  auto it = a.find(n);
  if (it == a.end()) return fallback;
  if (it->second.kind == XRMM_ATTR_FLOAT) return it->second.f;
  if (it->second.kind == XRMM_ATTR_INT) return double(it->second.i);
  const std::string& s = it->second.s;
  size_t used = 0;
  double v = 0;
  try {
    v = std::stod(s, &used);
  } catch (...) {
    used = 0;
  }
  if (s.empty() || used != s.size()) throw Invalid("Invalid numeric attribute " + n);
  return v;
}

std::string attr_str(const Attrs& a, const std::string& n, const std::string& fallback) {
  auto it = a.find(n);
  return it == a.end() || it->second.kind != XRMM_ATTR_STRING ? fallback : it->second.s;
}

// activation_lower (complex_plan.cpp:55)
int activation_code(const std::string& name) {
  static const std::map<std::string, int> m = {{"none", 0}, {"", 0}, {"identity", 0}, {"relu", 1}, {"silu", 2},
                                               {"swish", 2}, {"gelu", 3}, {"tanh", 4}, {"sigmoid", 5}, {"swiglu", 6}};
  auto it = m.find(name);
  if (it == m.end()) throw Invalid("Unknown fused activation: " + name);
  return it->second;
}

struct Plan {
  const OpContract* contract = nullptr;
  std::map<std::string, Tensor> in;   // present inputs by port name
  std::vector<Tensor> outputs;        // planned, in canonical order
  int64_t K = 0, N = 0, Nq = 0, Nkv = 0, M = 0;
  int32_t bits = 4, block_size = 32, act = 2, dtype = XRMM_F32, zp_dtype = XRMM_UNSPECIFIED;
  float eps = 1e-5f;
  // MatMulBnb4
  int32_t quant_type = 1, trans_b = 1;
  // QMoE
  int64_t T = 0, H = 0, E = 0, F1 = 0, I = 0;
  int32_t k = 1, fusion = 0, has_limit = 0;
  float alpha = 1.f, beta = 0.f, limit = 0.f;
  // GatherBlockQuantized
  int64_t rows = 0, pcols = 0, n_idx = 0;
  int32_t idx_dtype = XRMM_I64;
  std::map<std::string, std::vector<int64_t>> out_shape;  // planned output shapes by port

  const Tensor* get(const char* n) const {
    auto it = in.find(n);
    return it == in.end() ? nullptr : &it->second;
  }
};

void check(bool ok, const std::string& reason) {
  if (!ok) throw Invalid(reason);
}

void expect_shape(const Tensor* t, const std::vector<int64_t>& want) {
  if (!t) return;
  if (t->shape != want) {
    std::ostringstream o;
    o << t->name << " must have shape [";
    for (size_t i = 0; i < want.size(); ++i) o << (i ? "," : "") << want[i];
    o << "]";
    throw Invalid(o.str());
  }
}

// Planned outputs in contract order from p.out_shape (optional ones only when
// requested), then the requested-output checks that select storage dtypes
// (planner.cpp:86-93). Output dtypes follow their type variable.
void finish_outputs(Plan& p, const xrmm_request* q) {
  const OpContract& c = *p.contract;
  if (q->n_requested_outputs < 0 || (q->n_requested_outputs > 0 && !q->requested_outputs)) throw Invalid("Invalid requested-output list");
  std::vector<Tensor> requested;
  for (int32_t i = 0; i < q->n_requested_outputs; ++i) requested.push_back(from_c(q->requested_outputs[i], false));
  for (const auto& pt : c.outputs) {
    const bool asked = std::any_of(requested.begin(), requested.end(), [&](const Tensor& t) { return t.name == pt.name; });
    if ((pt.optional && !asked) || (!requested.empty() && !asked)) continue;
    Tensor t;
    t.name = pt.name;
    t.dtype = t.storage = p.dtype;
    t.shape = p.out_shape.at(pt.name);
    p.outputs.push_back(t);
  }
  for (const auto& pt : c.outputs)
    if (!pt.optional && std::none_of(p.outputs.begin(), p.outputs.end(), [&](const Tensor& t) { return t.name == pt.name; }))
      throw Invalid(std::string("Missing required frozen-contract output: ") + pt.name);
  if (!requested.empty()) {
    check(requested.size() == p.outputs.size(), "Requested output count differs from plan");
    for (size_t i = 0; i < p.outputs.size(); ++i) {
      const Tensor& w = requested[i];
      Tensor& t = p.outputs[i];
      check(w.name == t.name && w.dtype == t.dtype, "Requested output name/type differs from plan");
      check(w.shape.size() == t.shape.size(), "Requested output rank differs from plan");
      check(w.shape == t.shape, "Requested output shape differs from plan");
      t.storage = w.storage;
    }
  }
}

// MatMulBnb4 (complex_plan.cpp:117-120): K defaults to A's last dimension,
// N required, block_size 32, quant_type 1 (NF4), transB 1.
void plan_bnb4(Plan& p, const Attrs& a) {
  const Tensor& A = p.in.at("aT");
  p.dtype = A.dtype;
  p.K = attr_int(a, "K", A.shape.back());
  p.N = attr_int(a, "N", 0);
  p.block_size = int32_t(attr_int(a, "block_size", 32));
  p.quant_type = int32_t(attr_int(a, "quant_type", 1));
  p.trans_b = int32_t(attr_int(a, "transB", 1));
  check(p.K > 0 && p.block_size > 0, "Invalid packed matmul geometry");
  check(p.N > 0, "Packed matmul N required");
  check(p.quant_type == 0 || p.quant_type == 1, "MatMulBnb4 quant_type must be 0 (FP4) or 1 (NF4)");
  check(A.shape.back() == p.K, "aT's last dimension must equal K");
  p.M = A.shape[0];
  check(int64_t(numel(p.in.at("bT").shape)) >= (p.N * p.K + 1) / 2, "bT holds fewer than N*K codes");
  check(int64_t(numel(p.in.at("absmaxT").shape)) >= (p.N * p.K + p.block_size - 1) / p.block_size,
        "absmaxT holds fewer than ceil(N*K/block_size) scales");
  p.out_shape["yT"] = {p.M, p.N};
}

// QMoE (complex_plan.cpp:121-128), with the reference's messages.
void plan_qmoe(Plan& p, const Attrs& a) {
  const Tensor& x = p.in.at("inputT");
  const Tensor& router = p.in.at("routerT");
  const Tensor& fc1 = p.in.at("fc1T");
  const Tensor& fc2 = p.in.at("fc2T");
  const Tensor& s1 = p.in.at("fc1ScalesT");
  const Tensor& s2 = p.in.at("fc2ScalesT");
  p.dtype = x.dtype;
  p.k = int32_t(attr_int(a, "k", 1));
  const int64_t sparse = attr_int(a, "use_sparse_mixer", 0);
  p.fusion = int32_t(attr_int(a, "swiglu_fusion", 0));
  p.bits = int32_t(attr_int(a, "expert_weight_bits", 4));
  p.block_size = int32_t(attr_int(a, "block_size", 0));
  const int64_t prepacked = attr_int(a, "weights_prepacked", -1);
  p.act = activation_code(attr_str(a, "activation_type", "relu"));
  p.alpha = float(attr_num(a, "activation_alpha", 1));
  p.beta = float(attr_num(a, "activation_beta", 0));
  p.limit = float(attr_num(a, "swiglu_limit", 0));
  p.has_limit = a.count("swiglu_limit") ? 1 : 0;
  p.H = x.shape.empty() ? 0 : x.shape.back();
  p.E = router.shape[1];
  p.F1 = fc1.shape[1];
  const int64_t fusion = p.act == 6 && p.fusion ? 2 : 1;
  p.I = p.F1 / fusion;
  check((x.shape.size() == 2 || x.shape.size() == 3) && p.H > 0 && p.k >= 1 && p.k <= p.E && sparse == 0,
        "Invalid MoE input or routing geometry");
  p.T = int64_t(numel(x.shape) / uint64_t(p.H));
  check(router.shape[0] == p.T && fc1.shape[0] == p.E && fc2.shape[0] == p.E && fc2.shape[1] == p.H &&
            p.F1 % fusion == 0,
        "Invalid MoE weight geometry");
  check((p.bits == 4 || p.bits == 8) && (prepacked == -1 || prepacked == 0) && attr_str(a, "quant_type", "int") == "int",
        "Unsupported QMoE integer layout");
  check((p.act == 1 && p.fusion == 0) || (p.act == 6 && p.fusion == 1), "Invalid quantized SwiGLU fusion");
  check(fc1.shape[2] * (8 / p.bits) == p.H && fc2.shape[2] * (8 / p.bits) == p.I, "Invalid packed expert projection");
  const int32_t bs = p.block_size;
  check(bs == 0 || (bs >= 16 && (bs & (bs - 1)) == 0 && p.H % bs == 0 && p.I % bs == 0),
        "Invalid quantized expert block size");
  for (const Tensor* sc : {&s1, &s2}) {
    const Tensor& w = sc == &s1 ? fc1 : fc2;
    const int64_t cols = sc == &s1 ? p.H : p.I;
    check(int(sc->shape.size()) == (bs ? 3 : 2) && sc->shape[0] == p.E && sc->shape[1] == w.shape[1] &&
              (!bs || sc->shape[2] == cols / bs),
          "Invalid quantized expert scales");
  }
  p.out_shape["outputT"] = x.shape;
}

// GatherBlockQuantized (complex_plan.cpp:129): bits 4 / 8, block_size a power
// of two >= 16, gather_axis 0, quantize_axis 1; output [indices, width] in the
// scales' dtype.
void plan_gbq(Plan& p, const Attrs& a, const std::map<std::string, int32_t>& vars) {
  const Tensor& data = p.in.at("dataT");
  const Tensor& idx = p.in.at("indicesT");
  const Tensor& sc = p.in.at("scalesT");
  p.bits = int32_t(attr_int(a, "bits", 4));
  p.block_size = int32_t(attr_int(a, "block_size", 128));
  const int64_t gather_axis = attr_int(a, "gather_axis", 0), quantize_axis = attr_int(a, "quantize_axis", 1);
  const int32_t bs = p.block_size;
  check((p.bits == 4 || p.bits == 8) && bs >= 16 && (bs & (bs - 1)) == 0 && gather_axis == 0 && quantize_axis == 1,
        "Unsupported GatherBlockQuantized geometry");
  p.dtype = sc.dtype;
  p.idx_dtype = idx.dtype;
  p.rows = data.shape[0];
  p.pcols = data.shape[1];
  p.n_idx = idx.shape[0];
  const int64_t width = p.pcols * (8 / p.bits), blocks = (width + bs - 1) / bs;
  expect_shape(&sc, {p.rows, blocks});
  expect_shape(p.get("zeroPointsT"), {p.rows, (blocks * p.bits + 7) / 8});
  (void)vars;
  p.out_shape["outputT"] = {p.n_idx, width};
}

Plan make_plan(const xrmm_request* q) {
  if (!q || !q->operation) throw Invalid("Missing request");
  Plan p;
  for (const auto& c : contracts())
    if (c.operation == std::string(q->operation)) p.contract = &c;
  if (!p.contract) throw Invalid(std::string("Unsupported extended operator: ") + q->operation);
  const OpContract& c = *p.contract;

  // ---- contract validation of inputs (contracts.cpp:14)
  if (q->n_inputs < 0 || (q->n_inputs > 0 && !q->inputs)) throw Invalid("Invalid input list");
  std::map<std::string, int32_t> vars;
  auto port_check = [&](const Port& port, const Tensor& t) {
    if ((port.mask & (1u << t.dtype)) == 0) throw Invalid("Logical dtype outside frozen contract: " + t.name);
    if (port.rank >= 0 && int(t.shape.size()) != port.rank) throw Invalid("Rank outside frozen contract: " + t.name);
    if (port.var[0] >= 'A' && port.var[0] <= 'Z') {
      auto prior = vars.find(port.var);
      if (prior != vars.end() && prior->second != t.dtype)
        throw Invalid(std::string("Type variable differs between tensors: ") + port.var);
      vars[port.var] = t.dtype;
    }
  };
  for (int32_t i = 0; i < q->n_inputs; ++i) {
    Tensor t = from_c(q->inputs[i], true);
    const Port* port = nullptr;
    for (const auto& pt : c.inputs)
      if (t.name == pt.name) port = &pt;
    if (!port) throw Invalid("Unknown input outside frozen contract: " + t.name);
    if (p.in.count(t.name)) throw Invalid("Duplicate or unnamed extended input");
    port_check(*port, t);
    p.in[t.name] = t;
  }
  for (const auto& pt : c.inputs)
    if (!pt.optional && !p.in.count(pt.name)) throw Invalid(std::string("Missing required frozen-contract input: ") + pt.name);

  const Attrs a = merged_attrs(*q);
  if (c.op == OP_BNB4 || c.op == OP_QMOE || c.op == OP_GBQ) {
    if (c.op == OP_BNB4) plan_bnb4(p, a);
    if (c.op == OP_QMOE) plan_qmoe(p, a);
    if (c.op == OP_GBQ) plan_gbq(p, a, vars);
    finish_outputs(p, q);
    return p;
  }

  // ---- attributes (complex_plan.cpp:118)
  const Tensor& A = p.in.at("aT");
  check(!A.shape.empty(), "Rank-one or greater tensor required");
  p.dtype = A.dtype;
  p.K = attr_int(a, "K", A.shape.back());
  p.N = attr_int(a, "N", 0);
  p.block_size = int32_t(attr_int(a, "block_size", 32));
  p.bits = int32_t(attr_int(a, "bits", 4));
  p.eps = float(attr_num(a, "epsilon", c.op == xrmm::OP_QKV ? 1e-6 : 1e-5));
  p.act = activation_code(attr_str(a, "activation", "silu"));
  check(p.K > 0 && p.block_size > 0, "Invalid packed matmul geometry");
  check(p.bits == 2 || p.bits == 4 || p.bits == 8, "bits must be 2, 4 or 8");
  if (c.op == xrmm::OP_QKV) {
    p.Nq = attr_int(a, "Nq", 0);
    p.Nkv = attr_int(a, "Nkv", 0);
    check(p.Nq > 0 && p.Nkv > 0, "Nq and Nkv must be positive");
  } else {
    check(p.N > 0, "Packed matmul N required");
  }

  // ---- geometry of the packed tensors (stricter than the reference)
  check(A.shape.back() == p.K, "aT's last dimension must equal K");
  p.M = int64_t(numel(A.shape) / uint64_t(p.K));
  const int64_t kb = (p.K + p.block_size - 1) / p.block_size;
  const int64_t blob = (int64_t(p.block_size) * p.bits + 7) / 8;
  const int64_t zrow = (kb * p.bits + 7) / 8;
  auto projection = [&](const char* b, const char* s, const char* z, int64_t n) {
    expect_shape(p.get(b), {n, kb, blob});
    expect_shape(p.get(s), {n, kb});
    if (const Tensor* zt = p.get(z)) expect_shape(zt, zt->dtype == XRMM_U8 ? std::vector<int64_t>{n, zrow} : std::vector<int64_t>{n, kb});
  };
  if (c.op == xrmm::OP_MATMUL) {
    projection("bT", "scalesT", "zeroPointsT", p.N);
    expect_shape(p.get("biasT"), {p.N});
  } else if (c.op == xrmm::OP_MLP) {
    projection("gateBT", "gateScalesT", "gateZeroPointsT", p.N);
    projection("upBT", "upScalesT", "upZeroPointsT", p.N);
    expect_shape(p.get("gateBiasT"), {p.N});
    expect_shape(p.get("upBiasT"), {p.N});
  } else {
    projection("qBT", "qScalesT", "qZeroPointsT", p.Nq);
    projection("kBT", "kScalesT", "kZeroPointsT", p.Nkv);
    projection("vBT", "vScalesT", "vZeroPointsT", p.Nkv);
  }
  expect_shape(p.get("skipT"), A.shape);
  expect_shape(p.get("normScaleT"), {p.K});
  auto zp = vars.find("T3");
  p.zp_dtype = zp == vars.end() ? XRMM_UNSPECIFIED : zp->second;

  // ---- outputs (complex_plan.cpp:66-72,119)
  auto last = [&](int64_t n) {
    auto sh = A.shape;
    sh.back() = n;
    return sh;
  };
  for (const auto& pt : c.outputs) {
    const std::string nm = pt.name;
    p.out_shape[nm] = nm == "residualT" ? A.shape : nm == "qT" ? last(p.Nq) : (nm == "kT" || nm == "vT") ? last(p.Nkv) : last(p.N);
  }
  finish_outputs(p, q);
  return p;
}

void fill_desc(const Tensor& t, xrmm_tensor_desc* d) {
  std::memset(d, 0, sizeof(*d));
  std::snprintf(d->name, sizeof(d->name), "%s", t.name.c_str());
  d->dtype = t.dtype;
  d->storage_dtype = t.storage;
  d->rank = int32_t(t.shape.size());
  for (size_t i = 0; i < t.shape.size(); ++i) d->shape[i] = t.shape[i];
  d->nbytes = numel(t.shape) * dtype_bytes(t.storage);
}

// ---- storage <-> logical conversion (planner.cpp:27 logical_bits, :51-66)

// Element j of `src` (storage dtype `from`) written as dtype `to` into dst.
// Float pairs convert with one IEEE round-to-nearest-even; integer pairs copy
// the low bytes (sign-extending signed sources), and a narrowing that loses
// information is an error on readback (`strict`).
void convert(const uint8_t* src, int32_t from, uint8_t* dst, int32_t to, uint64_t n, bool strict) {
  if (from == to) {
    std::memcpy(dst, src, n * dtype_bytes(from));
    return;
  }
  if (floating(from)) {
    for (uint64_t j = 0; j < n; ++j) {
      if (from == XRMM_F32) {
        float x;
        std::memcpy(&x, src + 4 * j, 4);
        const _Float16 h = static_cast<_Float16>(x);
        std::memcpy(dst + 2 * j, &h, 2);
      } else {
        _Float16 h;
        std::memcpy(&h, src + 2 * j, 2);
        const float x = static_cast<float>(h);
        std::memcpy(dst + 4 * j, &x, 4);
      }
    }
    return;
  }
  const uint32_t fb = dtype_bytes(from), tb = dtype_bytes(to);
  const bool fsigned = from == XRMM_I64 || from == XRMM_I32 || from == XRMM_I16 || from == XRMM_I8;
  const bool tsigned = to == XRMM_I64 || to == XRMM_I32 || to == XRMM_I16 || to == XRMM_I8;
  for (uint64_t j = 0; j < n; ++j) {
    uint64_t v = 0;
    std::memcpy(&v, src + fb * j, fb);
    if (fsigned && fb < 8 && (v >> (fb * 8 - 1)) & 1) v |= ~uint64_t(0) << (fb * 8);
    if (strict && tb < 8) {
      uint64_t back = v & ((uint64_t(1) << (tb * 8)) - 1);
      if (tsigned && (back >> (tb * 8 - 1)) & 1) back |= ~uint64_t(0) << (tb * 8);
      if (back != v) throw Device("Output value does not fit requested physical storage");
    }
    std::memcpy(dst + tb * j, &v, tb);
  }
}

void hip_check(hipError_t e, const char* where) {
  if (e != hipSuccess) throw Device(std::string(where) + ": " + hipGetErrorString(e));
}

// Whether a binary16 weight (code - z) * scale of a float16 request could leave
// the binary16 range (|w| > 65504), where the reference's float32 weight
// (complex_kernel.glsl:80) stays finite. The fast kernels that stage binary16
// weights would saturate such weights to +-Inf, so the run then uses only
// kernels that keep weights in float32.
bool weights_need_float32(const Plan& p) {
  const int op = p.contract->op;
  if (p.dtype != XRMM_F16 || (op != xrmm::OP_MATMUL && op != xrmm::OP_QKV && op != xrmm::OP_MLP)) return false;
  static const char* const kMatMul[][2] = {{"scalesT", "zeroPointsT"}};
  static const char* const kQkv[][2] = {{"qScalesT", "qZeroPointsT"}, {"kScalesT", "kZeroPointsT"}, {"vScalesT", "vZeroPointsT"}};
  static const char* const kMlp[][2] = {{"gateScalesT", "gateZeroPointsT"}, {"upScalesT", "upZeroPointsT"}};
  const char* const(*ports)[2] = op == xrmm::OP_MATMUL ? kMatMul : op == xrmm::OP_QKV ? kQkv : kMlp;
  const int nports = op == xrmm::OP_MATMUL ? 1 : op == xrmm::OP_QKV ? 3 : 2;
  const double code_max = double((1 << p.bits) - 1);
  auto max_abs = [](const Tensor& t) {
    const uint64_t n = numel(t.shape);
    std::vector<float> v(n);
    convert(t.data, t.storage, reinterpret_cast<uint8_t*>(v.data()), XRMM_F32, n, false);
    double m = 0;
    for (float x : v)
      if (std::fabs(double(x)) > m) m = std::fabs(double(x));  // NaN compares false: a NaN weight is NaN either way
    return m;
  };
  for (int i = 0; i < nports; ++i) {
    const Tensor* s = p.get(ports[i][0]);
    if (!s || !numel(s->shape)) continue;
    const Tensor* z = p.get(ports[i][1]);
    double zdiff = double(1 << (p.bits - 1));  // implicit midpoint
    if (z && z->dtype == XRMM_U8) zdiff = code_max;
    else if (z) zdiff = max_abs(*z) + code_max;
    if (max_abs(*s) * zdiff > 65504.0) return true;
  }
  return false;
}

}  // namespace

struct xrmm_op {
  Plan plan;
  xrmm_options options{};
  int device = -1;
  hipStream_t stream = nullptr;
  hipEvent_t ev_start = nullptr, ev_end = nullptr;
  uint8_t* arena = nullptr;
  uint64_t arena_bytes = 0;
  std::map<std::string, void*> in_dev;  // device copies of present inputs
  std::vector<void*> out_dev;           // device outputs in plan order
  void* workspace = nullptr;            // QMoE workspace / GatherBlockQuantized status word
  void* packed = nullptr;               // MatMulNBits prefill: B prepacked at prepare (xrmm_prepack_weights)
  uint64_t workspace_bytes = 0;
  bool closed = false, executed = false, poisoned = false, has_gpu = false;
  bool exact_weights = false;  // weights_need_float32 at prepare
  double execution_ms = 0, gpu_ms = 0;
  std::string kernel, device_name, info_json;

  void open() const {
    if (closed) throw Device("Extended native operator is closed");
    if (poisoned) throw Device("Extended native operator failed and must be closed");
  }

  void release() noexcept {
    if (stream) (void)hipStreamSynchronize(stream);
    if (arena) (void)hipFree(arena);
    if (packed) (void)hipFree(packed);
    packed = nullptr;
    if (ev_start) (void)hipEventDestroy(ev_start);
    if (ev_end) (void)hipEventDestroy(ev_end);
    if (stream) (void)hipStreamDestroy(stream);
    arena = nullptr;
    ev_start = ev_end = nullptr;
    stream = nullptr;
    in_dev.clear();
    out_dev.clear();
    closed = true;
  }

  const void* dptr(const char* n) const {
    auto it = in_dev.find(n);
    return it == in_dev.end() ? nullptr : it->second;
  }
  void* optr(const char* n) const {
    for (size_t i = 0; i < plan.outputs.size(); ++i)
      if (plan.outputs[i].name == n) return out_dev[i];
    return nullptr;
  }

  // Enqueue the operator through the zero-copy entry points.
  int enqueue() {
    const xrmm::ExactWeightsScope exact(exact_weights);
    const Plan& p = plan;
    void* s = stream;
    const int32_t zd = p.zp_dtype;
    switch (p.contract->op) {
      case OP_BNB4:
        return xrmm_matmul_bnb4(dptr("aT"), dptr("bT"), dptr("absmaxT"), optr("yT"), p.M, p.K, p.N, p.block_size,
                                p.quant_type, p.trans_b, p.dtype, s);
      case OP_QMOE:
        return xrmm_qmoe(dptr("inputT"), dptr("routerT"), dptr("fc1T"), dptr("fc1ScalesT"), dptr("fc2T"),
                         dptr("fc2ScalesT"), optr("outputT"), workspace, int64_t(workspace_bytes), p.T, p.H, p.E, p.F1,
                         p.k, p.bits, p.block_size, p.act, p.fusion, p.alpha, p.beta, p.limit, p.has_limit, s);
      case OP_GBQ: {
        // the status word starts at zero for every run (the kernels only raise it)
        const hipError_t e = hipMemsetAsync(workspace, 0, 4, stream);
        if (e != hipSuccess) return xrmm::set_status(XRMM_EDEVICE, std::string("hipMemsetAsync: ") + hipGetErrorString(e));
        return xrmm_gather_block_quantized(dptr("dataT"), dptr("indicesT"), p.idx_dtype, dptr("scalesT"),
                                           dptr("zeroPointsT"), optr("outputT"), workspace, p.rows, p.pcols, p.n_idx,
                                           p.bits, p.block_size, s);
      }
      case xrmm::OP_MATMUL:
        if (packed)
          return xrmm_matmul_nbits_prepacked(dptr("aT"), packed, dptr("scalesT"), dptr("zeroPointsT"),
                                             dptr("zeroPointsT") ? zd : XRMM_UNSPECIFIED, dptr("biasT"), optr("yT"), p.M,
                                             p.K, p.N, p.bits, p.block_size, p.dtype, s);
        if (workspace)
          return xrmm_matmul_nbits_ws(dptr("aT"), dptr("bT"), dptr("scalesT"), dptr("zeroPointsT"),
                                      dptr("zeroPointsT") ? zd : XRMM_UNSPECIFIED, dptr("biasT"), optr("yT"), p.M, p.K,
                                      p.N, p.bits, p.block_size, p.dtype, workspace, int64_t(workspace_bytes), s);
        return xrmm_matmul_nbits(dptr("aT"), dptr("bT"), dptr("scalesT"), dptr("zeroPointsT"), dptr("zeroPointsT") ? zd : XRMM_UNSPECIFIED,
                                 dptr("biasT"), optr("yT"), p.M, p.K, p.N, p.bits, p.block_size, p.dtype, s);
      case xrmm::OP_MLP: {
        const bool z = dptr("gateZeroPointsT") || dptr("upZeroPointsT");
        return xrmm_matmul_nbits_mlp_ws(dptr("aT"), dptr("skipT"), dptr("normScaleT"), dptr("gateBT"),
                                        dptr("gateScalesT"), dptr("gateZeroPointsT"), dptr("gateBiasT"), dptr("upBT"),
                                        dptr("upScalesT"), dptr("upZeroPointsT"), dptr("upBiasT"),
                                        z ? zd : XRMM_UNSPECIFIED, optr("yT"), optr("residualT"), p.M, p.K, p.N, p.bits,
                                        p.block_size, p.eps, p.act, p.dtype, workspace, int64_t(workspace_bytes), s);
      }
      default: {
        const bool z = dptr("qZeroPointsT") || dptr("kZeroPointsT") || dptr("vZeroPointsT");
        return xrmm_matmul_nbits_qkv_ws(dptr("aT"), dptr("skipT"), dptr("normScaleT"), dptr("qBT"), dptr("qScalesT"),
                                        dptr("qZeroPointsT"), dptr("kBT"), dptr("kScalesT"), dptr("kZeroPointsT"),
                                        dptr("vBT"), dptr("vScalesT"), dptr("vZeroPointsT"), z ? zd : XRMM_UNSPECIFIED,
                                        optr("qT"), optr("kT"), optr("vT"), optr("residualT"), p.M, p.K, p.Nq, p.Nkv,
                                        p.bits, p.block_size, p.eps, p.dtype, workspace, int64_t(workspace_bytes), s);
      }
    }
  }
};

namespace {

// Runs f and converts its exception class into the ABI status
// (std::invalid_argument -> XRMM_EINVAL, std::runtime_error -> XRMM_EDEVICE).
template <class F>
int guarded(F&& f) {
  try {
    f();
    return xrmm::set_status(XRMM_OK, "");
  } catch (const Invalid& e) {
    return xrmm::set_status(XRMM_EINVAL, e.what());
  } catch (const Device& e) {
    return xrmm::set_status(XRMM_EDEVICE, e.what());
  } catch (const std::bad_alloc&) {
    return xrmm::set_status(XRMM_EDEVICE, "host allocation failed");
  } catch (const std::exception& e) {
    return xrmm::set_status(XRMM_EINVAL, e.what());
  }
}

uint64_t align256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

}  // namespace

extern "C" {

void xrmm_default_options(xrmm_options* o) {
  if (!o) return;
  o->profiling = 0;
  o->timeout_ns = 15000000000ULL;
  o->memory_limit_bytes = 268435456ULL;
}

int xrmm_plan(const xrmm_request* request, xrmm_tensor_desc* outputs, int32_t capacity, int32_t* n_outputs) {
  return (guarded([&] {
    Plan p = make_plan(request);
    if (n_outputs) *n_outputs = int32_t(p.outputs.size());
    if (outputs) {
      if (capacity < int32_t(p.outputs.size())) throw Invalid("Output descriptor capacity too small");
      for (size_t i = 0; i < p.outputs.size(); ++i) fill_desc(p.outputs[i], outputs + i);
    }
  }));
}

int xrmm_prepare(const xrmm_request* request, const xrmm_options* options, xrmm_op** out) {
  return (guarded([&] {
    if (!out) throw Invalid("Missing operator handle");
    *out = nullptr;
    xrmm_options o;
    xrmm_default_options(&o);
    if (options) o = *options;
    if (!o.timeout_ns || !o.memory_limit_bytes) throw Invalid("Positive extended runtime limits required");
    auto op = std::make_unique<xrmm_op>();
    op->options = o;
    op->plan = make_plan(request);
    Plan& p = op->plan;

    // byte counts (planner.cpp:41) and the memory limit over device bytes
    uint64_t total = 0;
    for (auto& kv : p.in) {
      const Tensor& t = kv.second;
      const uint64_t n = numel(t.shape);
      if (t.nbytes != n * dtype_bytes(t.storage) || (n && !t.data))
        throw Invalid("Extended input byte count mismatch: " + t.name);
      total += align256(n * dtype_bytes(t.dtype));
    }
    for (const Tensor& t : p.outputs) total += align256(numel(t.shape) * dtype_bytes(t.dtype));
    uint64_t ws = 0;
    if (p.contract->op == OP_QMOE) ws = uint64_t(xrmm_qmoe_workspace_bytes(p.T, p.k, p.H, p.I));
    if (p.contract->op == OP_GBQ) ws = 4;
    total += align256(ws);
    if (total > o.memory_limit_bytes) throw Invalid("Extended heap memory limit exceeded");
    // The MatMulNBits workspace (split K, the float32-arithmetic GEMM) and
    // the normalised-activation workspace of the Qkv / Mlp prefill GEMMs are
    // performance options, not part of the request's memory: each is
    // reserved only when it fits the limit beside the data, and the call runs
    // without it otherwise. Weights beyond binary16 keep the MatMulNBits one
    // (for the float32-arithmetic GEMM).
    {
      const bool exact = weights_need_float32(p);
      const xrmm::ExactWeightsScope scope(exact);
      uint64_t opt = 0;
      if (p.contract->op == xrmm::OP_MATMUL)
        opt = uint64_t(xrmm_matmul_nbits_workspace_bytes(p.M, p.K, p.N, p.bits, p.block_size, p.dtype));
      else if (!exact && (p.contract->op == xrmm::OP_QKV || p.contract->op == xrmm::OP_MLP))
        opt = uint64_t(xrmm_matmul_nbits_fused_workspace_bytes(
            p.contract->op, p.M, p.K, p.contract->op == xrmm::OP_QKV ? p.Nq : p.N, p.Nkv, p.bits, p.block_size,
            p.dtype, p.in.count("skipT") ? 1 : 0, p.in.count("normScaleT") ? 1 : 0));
      if (opt && total + align256(opt) <= o.memory_limit_bytes) {
        ws = opt;
        total += align256(opt);
      }
    }

    hip_check(hipGetDevice(&op->device), "hipGetDevice");
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, op->device), "hipGetDeviceProperties");
    op->device_name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    op->arena_bytes = total;
    if (total) hip_check(hipMalloc(reinterpret_cast<void**>(&op->arena), total), "hipMalloc");
    hip_check(hipStreamCreateWithFlags(&op->stream, hipStreamNonBlocking), "hipStreamCreate");
    hip_check(hipEventCreate(&op->ev_start), "hipEventCreate");
    hip_check(hipEventCreate(&op->ev_end), "hipEventCreate");

    // upload: inputs converted to their logical dtype, one staging copy each
    uint64_t off = 0;
    std::vector<uint8_t> staging;
    for (auto& kv : p.in) {
      const Tensor& t = kv.second;
      const uint64_t n = numel(t.shape), bytes = n * dtype_bytes(t.dtype);
      void* d = op->arena + off;
      op->in_dev[t.name] = d;
      off += align256(bytes);
      if (!bytes) continue;
      const void* src = t.data;
      if (t.storage != t.dtype) {
        staging.resize(bytes);
        convert(t.data, t.storage, staging.data(), t.dtype, n, false);
        src = staging.data();
      }
      hip_check(hipMemcpyAsync(d, src, bytes, hipMemcpyHostToDevice, op->stream), "hipMemcpy (input)");
      hip_check(hipStreamSynchronize(op->stream), "hipStreamSynchronize");
    }
    for (const Tensor& t : p.outputs) {
      op->out_dev.push_back(op->arena + off);
      off += align256(numel(t.shape) * dtype_bytes(t.dtype));
    }
    op->workspace = ws ? op->arena + off : nullptr;
    op->workspace_bytes = ws;
    if (ws && p.contract->op == xrmm::OP_MATMUL) {  // the split-K counters start at zero (and stay there)
      hip_check(hipMemsetAsync(op->workspace, 0, ws, op->stream), "hipMemsetAsync (workspace)");
      hip_check(hipStreamSynchronize(op->stream), "hipStreamSynchronize");
    }
    const int32_t zk = p.zp_dtype;
    const int code = p.contract->op;
    const char* k = nullptr;
    if (code == OP_BNB4) {
      k = xrmm_matmul_bnb4_kernel(p.M, p.K, p.N, p.block_size, p.quant_type, p.trans_b, p.dtype);
    } else if (code == OP_QMOE) {
      k = xrmm_qmoe_kernel(p.T, p.H, p.E, p.F1, p.k, p.bits, p.block_size, p.act, p.fusion);
    } else if (code == OP_GBQ) {
      xrmm::GbqArgs g{};
      g.data = static_cast<const uint8_t*>(op->dptr("dataT"));
      g.out = static_cast<float*>(op->out_dev.empty() ? nullptr : op->out_dev[0]);
      g.pcols = p.pcols;
      g.bs = p.block_size;
      k = xrmm::gbq_fast_ok(g) ? "gbq_words" : "gbq_scalar";
    } else {
      op->exact_weights = weights_need_float32(p);
      const xrmm::ExactWeightsScope exact(op->exact_weights);
      const int64_t n0 = code == xrmm::OP_QKV ? p.Nq : p.N;
      k = xrmm::select_kernel_name(code, p.M, p.K, n0, p.bits, p.block_size, p.dtype, zk, op->workspace != nullptr);
      // prepare = upload / prepack: MatMulNBits requests that reach the 256 x
      // 256 prefill GEMM get their weights prepacked once, here, when the
      // copy fits the memory limit beside the arena
      const int64_t pk = code == xrmm::OP_MATMUL && k && std::strcmp(k, "gemm_q4_big") == 0
                             ? xrmm_prepacked_bytes(p.N, p.K, p.bits, p.block_size) : 0;
      if (pk > 0 && total + uint64_t(pk) <= o.memory_limit_bytes) {
        hip_check(hipMalloc(&op->packed, size_t(pk)), "hipMalloc (prepacked weights)");
        if (xrmm_prepack_weights(op->dptr("bT"), op->packed, p.N, p.K, p.bits, p.block_size, op->stream) != XRMM_OK)
          throw Device(std::string("prepack: ") + xrmm_last_error());
        hip_check(hipStreamSynchronize(op->stream), "hipStreamSynchronize");
        k = "gemm_q4_big_prepacked";
      }
    }
    op->kernel = k ? k : "generic";
    *out = op.release();
  }));
}

int xrmm_run(xrmm_op* op) {
  return (guarded([&] {
    if (!op) throw Invalid("Missing operator handle");
    op->open();
    op->executed = false;
    op->has_gpu = false;
    const auto t0 = std::chrono::steady_clock::now();
    try {
      hip_check(hipSetDevice(op->device), "hipSetDevice");
      hip_check(hipEventRecord(op->ev_start, op->stream), "hipEventRecord");
      const int rc = op->enqueue();
      if (rc != XRMM_OK) {
        const std::string why = xrmm_last_error();
        if (rc == XRMM_EINVAL) throw Invalid(why);
        throw Device(why);
      }
      hip_check(hipEventRecord(op->ev_end, op->stream), "hipEventRecord");
      // bounded wait (vulkan.cpp:115 waits on its fence with options.timeout_ns)
      const auto deadline = t0 + std::chrono::nanoseconds(op->options.timeout_ns);
      for (;;) {
        const hipError_t e = hipEventQuery(op->ev_end);
        if (e == hipSuccess) break;
        if (e != hipErrorNotReady) hip_check(e, "operator execution");
        if (std::chrono::steady_clock::now() > deadline) throw Device("Extended native operator timed out");
        std::this_thread::sleep_for(std::chrono::microseconds(20));
      }
      if (op->plan.contract->op == OP_GBQ) {  // failure code of the shader (vulkan.cpp:115)
        uint32_t code = 0;
        hip_check(hipMemcpy(&code, op->workspace, 4, hipMemcpyDeviceToHost), "hipMemcpy (status)");
        if (code) throw Device("GPU operator contract validation failed: code " + std::to_string(code));
      }
    } catch (...) {
      op->poisoned = true;
      throw;
    }
    op->execution_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (op->options.profiling) {
      float ms = 0;
      if (hipEventElapsedTime(&ms, op->ev_start, op->ev_end) == hipSuccess) {
        op->gpu_ms = ms;
        op->has_gpu = true;
      }
    }
    op->executed = true;
  }));
}

int xrmm_output_descs(const xrmm_op* op, xrmm_tensor_desc* outputs, int32_t capacity, int32_t* n_outputs) {
  return (guarded([&] {
    if (!op) throw Invalid("Missing operator handle");
    if (n_outputs) *n_outputs = int32_t(op->plan.outputs.size());
    if (outputs) {
      if (capacity < int32_t(op->plan.outputs.size())) throw Invalid("Output descriptor capacity too small");
      for (size_t i = 0; i < op->plan.outputs.size(); ++i) fill_desc(op->plan.outputs[i], outputs + i);
    }
  }));
}

int xrmm_read_outputs(xrmm_op* op, void* const* dst, const uint64_t* dst_bytes, int32_t n) {
  return (guarded([&] {
    if (!op) throw Invalid("Missing operator handle");
    op->open();
    if (!op->executed) throw Device("Run extended operator before readback");
    if (n != int32_t(op->plan.outputs.size())) throw Invalid("Requested output count mismatch");
    if (n && (!dst || !dst_bytes)) throw Invalid("Missing output buffers");
    std::vector<uint8_t> staging;
    hip_check(hipSetDevice(op->device), "hipSetDevice");
    for (int32_t i = 0; i < n; ++i) {
      const Tensor& t = op->plan.outputs[i];
      const uint64_t cnt = numel(t.shape), logical = cnt * dtype_bytes(t.dtype), stored = cnt * dtype_bytes(t.storage);
      if (dst_bytes[i] != stored || (stored && !dst[i])) throw Invalid("Output buffer size mismatch: " + t.name);
      if (!stored) continue;
      void* target = t.storage == t.dtype ? dst[i] : nullptr;
      if (!target) {
        staging.resize(logical);
        target = staging.data();
      }
      hip_check(hipMemcpyAsync(target, op->out_dev[i], logical, hipMemcpyDeviceToHost, op->stream), "hipMemcpy (output)");
      hip_check(hipStreamSynchronize(op->stream), "hipStreamSynchronize");
      if (t.storage != t.dtype) convert(staging.data(), t.dtype, static_cast<uint8_t*>(dst[i]), t.storage, cnt, true);
    }
  }));
}

const char* xrmm_info(xrmm_op* op) {
  if (!op) return "{}";
  std::ostringstream o;
  o.precision(17);
  o << "{\"backend\":\"hip\",\"test_only\":false,\"physical_qualification\":false,\"cpu_compute_fallback\":false,"
    << "\"extended\":true,\"operation\":\"" << op->plan.contract->operation << "\",\"closed\":" << (op->closed ? "true" : "false")
    << ",\"executed\":" << (op->executed ? "true" : "false") << ",\"execution_ms\":";
  if (op->executed) o << op->execution_ms; else o << "null";
  o << ",\"gpu_ms\":";
  if (op->has_gpu) o << op->gpu_ms; else o << "null";
  const Plan& pl = op->plan;
  const int pc = pl.contract->op;
  const bool work = pc == OP_QMOE ? pl.T > 0 : pc == OP_GBQ ? pl.n_idx > 0 : pl.M > 0;
  o << ",\"dispatch_count\":" << (op->executed && work ? 1 : 0) << ",\"persistent_bytes\":" << (op->closed ? 0 : op->arena_bytes)
    << ",\"device\":\"" << op->device_name << "\",\"kernel\":\"" << op->kernel << "\",\"outputs\":[";
  for (size_t i = 0; i < op->plan.outputs.size(); ++i) {
    const Tensor& t = op->plan.outputs[i];
    o << (i ? "," : "") << "{\"name\":\"" << t.name << "\",\"dtype\":\"" << dtype_name(t.dtype) << "\",\"storage_dtype\":\""
      << dtype_name(t.storage) << "\",\"shape\":[";
    for (size_t j = 0; j < t.shape.size(); ++j) o << (j ? "," : "") << t.shape[j];
    o << "]}";
  }
  o << "]}";
  op->info_json = o.str();
  return op->info_json.c_str();
}

int xrmm_close(xrmm_op* op) {
  return (guarded([&] {
    if (!op) throw Invalid("Missing operator handle");
    op->release();
  }));
}

void xrmm_destroy(xrmm_op* op) {
  if (!op) return;
  op->release();
  delete op;
}

}  // extern "C"
