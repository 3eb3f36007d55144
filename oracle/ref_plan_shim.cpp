// Test infrastructure (the oracle side): a C binding of the reference's own
// planner, xrgpu::operators::extended::plan (kernels/_shared/extended/
// planner.cpp:67, complex branch complex_plan.cpp:117-129, contract rows
// contracts.cpp / contract_data.h), compiled from the reference sources by
// oracle/Makefile into oracle/_ref/libref_plan.so. It takes the same request
// structure as xrmm_plan (include/xrmm.h), converts it to the reference's
// Request and writes the planned outputs in xrmm_plan's descriptor format, so
// a test hands one request to both planners and compares the answers (output
// names, dtypes, storage dtypes, shapes, and the messages of rejected
// requests). Only tests/ load it; the product never does.
#include <xrgpu/extended_operators.h>

#include <cstring>
#include <stdexcept>
#include <string>

#include "xrmm.h"

namespace x = xrgpu::operators;
namespace xe = xrgpu::operators::extended;

namespace {

x::Tensor to_ref(const xrmm_tensor& t) {
  x::Tensor r;
  r.name = t.name ? t.name : "";
  r.dtype = static_cast<x::DType>(t.dtype);
  r.storage_dtype = static_cast<x::DType>(t.storage_dtype);
  r.shape.assign(t.shape, t.shape + (t.rank > 0 ? t.rank : 0));
  if (t.data && t.nbytes) {
    const uint8_t* p = static_cast<const uint8_t*>(t.data);
    r.data.assign(p, p + t.nbytes);
  }
  return r;
}

void put_attrs(xe::Attributes& dst, const xrmm_attr* a, int32_t n) {
  for (int32_t i = 0; i < n; ++i) {
    const std::string k = a[i].key ? a[i].key : "";
    if (a[i].kind == XRMM_ATTR_INT) dst.integers[k] = a[i].i;
    else if (a[i].kind == XRMM_ATTR_FLOAT) dst.numbers[k] = a[i].f;
    else dst.strings[k] = a[i].s ? a[i].s : "";
  }
}

void message(char* buf, uint64_t cap, const char* what) {
  if (buf && cap) {
    std::strncpy(buf, what, cap - 1);
    buf[cap - 1] = 0;
  }
}

}  // namespace

// 0: planned (descriptors written), 1: std::invalid_argument, 2: any other
// exception; the exception's message goes to `msg`.
extern "C" int ref_plan(const xrmm_request* req, xrmm_tensor_desc* outs, int32_t capacity, int32_t* n_outputs,
                        char* msg, uint64_t msg_cap) {
  message(msg, msg_cap, "");
  *n_outputs = 0;
  try {
    xe::Request r;
    r.operation = req->operation ? req->operation : "";
    for (int32_t i = 0; i < req->n_inputs; ++i) r.inputs.push_back(to_ref(req->inputs[i]));
    for (int32_t i = 0; i < req->n_requested_outputs; ++i) r.requested_outputs.push_back(to_ref(req->requested_outputs[i]));
    put_attrs(r.attrs, req->attrs, req->n_attrs);
    put_attrs(r.args, req->args, req->n_args);
    const xe::ExtendedPlan p = xe::plan(r);
    int32_t n = 0;
    for (const x::Tensor& t : p.outputs) {
      if (n >= capacity) break;
      xrmm_tensor_desc& d = outs[n++];
      std::memset(&d, 0, sizeof d);
      std::strncpy(d.name, t.name.c_str(), XRMM_NAME_MAX - 1);
      d.dtype = static_cast<int32_t>(t.dtype);
      d.storage_dtype = static_cast<int32_t>(t.storage_dtype == x::DType::Unspecified ? t.dtype : t.storage_dtype);
      d.rank = static_cast<int32_t>(t.shape.size());
      uint64_t count = 1;
      for (size_t k = 0; k < t.shape.size() && k < XRMM_MAX_RANK; ++k) {
        d.shape[k] = t.shape[k];
        count *= static_cast<uint64_t>(t.shape[k]);
      }
      d.nbytes = count * x::dtype_bytes(static_cast<x::DType>(d.storage_dtype));
    }
    *n_outputs = n;
    return 0;
  } catch (const std::invalid_argument& e) {
    message(msg, msg_cap, e.what());
    return 1;
  } catch (const std::exception& e) {
    message(msg, msg_cap, e.what());
    return 2;
  }
}
