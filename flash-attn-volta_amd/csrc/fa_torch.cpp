// Autograd node of flash_attn / flash_attn_gqa in C++ (Python module
// flash_attn_volta._fa_torch), a client of the C ABI in fa_mi355x.h.
//
// The reference's autograd.Function (flash_attn_volta/autograd.py:19-59)
// is Python, and so is this package's (autograd.py).  A Python backward
// node makes torch's autograd engine thread take the GIL while the thread
// that called backward() waits for it, a hand-off that costs about as much
// host time as the whole fwd+bwd launch work of a small config.  This node
// runs its backward in C++ without the GIL.  Python keeps the argument
// checks and the per-signature launch plan (forward.py); a plan handed
// here (make_plan) holds the sizes, strides, scale and workspace sizes the
// two C calls need, and attn() runs the forward and records the node.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <optional>
#include <unordered_set>
#include <vector>

#include "fa_mi355x.h"

namespace {

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// Launch arguments of one call signature.  Plans live until the process
// ends (deduplicated by content), so a node's plan pointer never dangles.
struct Plan {
  int B, Sq, Sk, H, Hk, D;
  int gqa, causal, dtype;
  float scale;
  int64_t q_st[4], k_st[4], v_st[4], o_st[4];   // kernel strides, 0 for size-1 dims
  int64_t dq_st[4], dk_st[4];                   // contiguous gradients
  size_t fwd_ws;                                // fa_fwd_ws workspace, 0: plain forward
  size_t ws_split, ws_plain;                    // backward workspace, split schedule or not
};

constexpr size_t kPlanInts = 9 + 24 + 3;

std::mutex g_mu;
std::map<std::vector<int64_t>, std::unique_ptr<Plan>> g_plans;
std::unordered_set<int64_t> g_handles;

int64_t make_plan(const std::vector<int64_t> &v, double scale) {
  TORCH_CHECK(v.size() == kPlanInts, "make_plan: expected ", kPlanInts, " integers, got ", v.size());
  std::vector<int64_t> key(v);
  const float s = static_cast<float>(scale);
  int32_t bits;
  std::memcpy(&bits, &s, sizeof bits);
  key.push_back(bits);
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_plans.find(key);
  if (it != g_plans.end()) return reinterpret_cast<int64_t>(it->second.get());
  auto p = std::make_unique<Plan>();
  size_t i = 0;
  p->B = (int)v[i++]; p->Sq = (int)v[i++]; p->Sk = (int)v[i++];
  p->H = (int)v[i++]; p->Hk = (int)v[i++]; p->D = (int)v[i++];
  p->gqa = (int)v[i++]; p->causal = (int)v[i++]; p->dtype = (int)v[i++];
  for (int64_t *st : {p->q_st, p->k_st, p->v_st, p->o_st, p->dq_st, p->dk_st})
    for (int j = 0; j < 4; ++j) st[j] = v[i++];
  p->fwd_ws = (size_t)v[i++];
  p->ws_split = (size_t)v[i++];
  p->ws_plain = (size_t)v[i++];
  p->scale = s;
  const int64_t h = reinterpret_cast<int64_t>(p.get());
  g_handles.insert(h);
  g_plans.emplace(std::move(key), std::move(p));
  return h;
}

const Plan &plan_of(int64_t h) {
  std::lock_guard<std::mutex> lock(g_mu);
  TORCH_CHECK(g_handles.count(h), "flash_attn_volta._fa_torch: unknown plan handle");
  return *reinterpret_cast<const Plan *>(h);
}

void *stream_of(const Tensor &t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

bool aligned(const Tensor &t) { return (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) == 0; }

void check(int rc, const char *where) {
  TORCH_CHECK(rc == FA_OK, where, ": ", fa_strerror(rc), " (status ", rc, ")");
}

struct FlashAttnFn : public torch::autograd::Function<FlashAttnFn> {
  static Tensor forward(AutogradContext *ctx, const Tensor &q, const Tensor &k, const Tensor &v,
                        int64_t handle, bool split) {
    const Plan &p = *reinterpret_cast<const Plan *>(handle);
    const c10::DeviceGuard guard(q.device());
    Tensor out = at::empty({p.B, p.Sq, p.H, p.D}, q.options());
    Tensor lse = at::empty({p.B, p.H, p.Sq}, q.options().dtype(at::kFloat));
    void *stream = stream_of(q);
    if (p.fwd_ws) {
      Tensor ws = at::empty({(int64_t)p.fwd_ws}, q.options().dtype(at::kByte));
      check(fa_fwd_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                      lse.data_ptr<float>(), ws.data_ptr(), p.fwd_ws, p.B, p.Sq, p.Sk, p.H, p.Hk,
                      p.D, p.q_st, p.k_st, p.v_st, p.o_st, p.scale, p.causal, p.dtype, stream),
            "fa_fwd_ws");
    } else if (p.gqa) {
      check(fa_fwd_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                       lse.data_ptr<float>(), p.B, p.Sq, p.Sk, p.H, p.Hk, p.D, p.q_st, p.k_st,
                       p.v_st, p.o_st, p.scale, p.causal, p.dtype, stream),
            "fa_fwd_gqa");
    } else {
      check(fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr<float>(),
                   p.B, p.Sq, p.H, p.D, p.q_st, p.k_st, p.v_st, p.o_st, p.scale, p.causal, stream),
            "fa_fwd");
    }
    ctx->save_for_backward({q, k, v, out, lse});
    ctx->saved_data["plan"] = handle;
    ctx->saved_data["split"] = split;
    return out;
  }

  static variable_list backward(AutogradContext *ctx, variable_list grads) {
    const variable_list s = ctx->get_saved_variables();
    const Tensor &q = s[0], &k = s[1], &v = s[2], &out = s[3], &lse = s[4];
    const Plan &p = *reinterpret_cast<const Plan *>(ctx->saved_data["plan"].toInt());
    const bool split = ctx->saved_data["split"].toBool();
    const c10::DeviceGuard guard(q.device());
    // dO as the kernels read it: the forward's dtype, contiguous (the
    // plan's out strides), 16-byte aligned
    Tensor dout = grads[0];
    if (dout.scalar_type() != q.scalar_type()) dout = dout.to(q.scalar_type());
    dout = dout.contiguous();
    if (!aligned(dout)) dout = dout.clone(at::MemoryFormat::Contiguous);
    Tensor dq = at::empty({p.B, p.Sq, p.H, p.D}, q.options());
    // separate allocations, as the Python path's
    Tensor dk = at::empty({p.B, p.Sk, p.Hk, p.D}, q.options());
    Tensor dv = at::empty({p.B, p.Sk, p.Hk, p.D}, q.options());
    const size_t nb = split ? p.ws_split : p.ws_plain;
    Tensor ws = at::empty({(int64_t)nb}, q.options().dtype(at::kByte));
    void *stream = stream_of(q);
    if (p.gqa) {
      check(fa_bwd_gqa(dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                       lse.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                       ws.data_ptr(), nb, p.B, p.Sq, p.Sk, p.H, p.Hk, p.D, p.o_st, p.q_st,
                       p.k_st, p.v_st, p.o_st, p.dq_st, p.dk_st, p.dk_st, p.scale, p.causal,
                       p.dtype, stream),
            "fa_bwd_gqa");
    } else {
      check(fa_bwd(dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                   lse.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                   ws.data_ptr(), nb, p.B, p.Sq, p.H, p.D, p.o_st, p.q_st, p.k_st, p.v_st,
                   p.o_st, p.dq_st, p.dk_st, p.dk_st, p.scale, p.causal, stream),
            "fa_bwd");
    }
    return {dq, dk, dv, Tensor(), Tensor()};
  }
};

// The forward of plan `handle` on q, k, v (whose shapes, strides, dtype and
// device the caller matched to the plan), recording the backward node when
// any input requires grad.  None when a data pointer is not 16-byte
// aligned: the caller then takes its general path.
std::optional<Tensor> attn(int64_t handle, const Tensor &q, const Tensor &k, const Tensor &v,
                           bool split) {
  plan_of(handle);
  if (!aligned(q) || !aligned(k) || !aligned(v)) return std::nullopt;
  return FlashAttnFn::apply(q, k, v, handle, split);
}

}  // namespace

PYBIND11_MODULE(_fa_torch, m) {
  // This module calls the library's entry points with the argument lists of
  // the header it was compiled against; a library built from another ABI
  // version (the two .so files are built separately) would take them
  // without an error.  Refuse to load then: the Python autograd path, which
  // checks the version itself, takes over.
  if (fa_abi_version() != FA_ABI_VERSION) {
    PyErr_Format(PyExc_ImportError,
                 "_fa_torch was built for libfa_mi355x ABI %d, the loaded library has ABI %d: "
                 "rebuild both (flash_attn_volta.build)",
                 (int)FA_ABI_VERSION, (int)fa_abi_version());
    throw pybind11::error_already_set();
  }
  m.doc() = "C++ autograd node of flash_attn_volta's flash_attn / flash_attn_gqa";
  m.def("make_plan", &make_plan, "register a launch plan (ints, sm_scale) -> handle");
  m.def("attn", &attn, "forward of a plan, recording the C++ backward node");
  m.attr("PLAN_INTS") = (int64_t)kPlanInts;
}
