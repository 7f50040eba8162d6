// PyTorch functions of the training path (autograd) and the inference call (host code only).
//
// twopass_attention_train runs through Attention (q, k, v as given), and the timm drop-ins
// through QkvAttention (q, k, v = qkv[:, :, 0..2] of a [B, N, 3, H, D] projection).  Both
// keep the whole host side of one training call in C++:
//   forward   planner query, workspace, elsa_fwd with row state, out as [B, N, H, D]
//   backward  elsa_bwd writing dq, dk, dv into one [B, N, 3, H, D] gradient, and
//             elsa_dbias when the bias needs a gradient
// so that no Python runs between the launches and the backward needs no interpreter lock
// on autograd's device thread.  They mirror _TwopassAttentionAutograd / _TwopassQkvAutograd in
// attention_bwd.py (the Python twins, used for inputs that need a dense padded copy) and the
// reference's _TwopassAttentionAutograd (attention_bwd.py:842-905).  attention_forward is the
// inference call (twopass_attention) with the same host side in C++: one planner query, the
// workspace and elsa_fwd, without row state.
#include <ATen/hip/HIPContext.h>
#include <torch/extension.h>

#include <array>

#include "elsa_hip.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

int32_t code_of(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return ELSA_F16;
    case at::kBFloat16: return ELSA_BF16;
    case at::kFloat: return ELSA_F32;
    default: TORCH_CHECK(false, "supported dtypes are fp16, bf16, and fp32");
  }
  return -1;
}

void check(int rc, const char* what) {
  TORCH_CHECK(rc == ELSA_OK, what, " failed (status ", rc, "): ", elsa_last_error());
}

void* current_stream() { return at::hip::getCurrentHIPStream().stream(); }

elsa_layout layout_of(const at::Tensor& t) { return elsa_layout{t.stride(0), t.stride(1), t.stride(2)}; }

// The layout rules of the C ABI (a dense last dimension, strides in multiples of 8
// elements, a 16-byte aligned base); anything else is read from a dense copy.
at::Tensor operand(const at::Tensor& t) {
  const bool ok = t.stride(3) == 1 && t.stride(0) % 8 == 0 && t.stride(1) % 8 == 0 && t.stride(2) % 8 == 0 &&
                  t.stride(0) >= 0 && t.stride(1) >= 0 && t.stride(2) >= t.size(3) && t.stride(2) < (1 << 25) &&
                  reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
  return ok ? t : t.contiguous();
}

// bias: [1|B, 1|H, N, N], broadcast by zero strides
elsa_bias_desc bias_desc(const at::Tensor& bias) {
  elsa_bias_desc b{};
  b.dtype = ELSA_F32;
  if (!bias.defined()) return b;
  b.ptr = bias.data_ptr();
  b.dtype = code_of(bias.scalar_type());
  b.stride_b = bias.size(0) == 1 ? 0 : bias.stride(0);
  b.stride_h = bias.size(1) == 1 ? 0 : bias.stride(1);
  b.stride_q = bias.stride(2);
  b.stride_k = bias.stride(3);
  return b;
}

// [B, H, N, D] views of the q, k, v slices of a [B, N, 3, H, D] tensor
std::array<at::Tensor, 3> unbind_qkv(const at::Tensor& qkv) {
  const at::Tensor t = qkv.permute({2, 0, 3, 1, 4});
  return {t[0], t[1], t[2]};
}

at::Tensor bytes(const at::Tensor& like, size_t n) {
  return at::empty({static_cast<int64_t>(n)}, like.options().dtype(at::kByte));
}

struct FwdState {
  at::Tensor out, row_m, row_z;
};

// elsa_fwd on [B, H, N, D] operands (any layout the ABI accepts); out is written as
// [B, N, H, D] memory when out_bnhd, else dense.  With want_state the row state is stored too:
// the training forward's, a reference within 8 below the row maximum, z relative to it.
FwdState fwd_call(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& bias, bool causal,
                  int64_t summary_dtype, int64_t partition_len, int64_t q_chunk, bool out_bnhd,
                  bool want_state = true) {
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  FwdState st;
  st.out = out_bnhd ? at::empty({B, N, H, D}, q.options()).permute({0, 2, 1, 3}) : at::empty({B, H, N, D}, q.options());
  const auto f32 = q.options().dtype(at::kFloat);
  if (want_state) {
    st.row_m = at::empty({B * H, N}, f32);
    st.row_z = at::empty({B * H, N}, f32);
  }
  elsa_fwd_args a{};
  a.q = q.data_ptr();
  a.k = k.data_ptr();
  a.v = v.data_ptr();
  a.out = st.out.data_ptr();
  a.row_m = want_state ? st.row_m.data_ptr<float>() : nullptr;
  a.row_z = want_state ? st.row_z.data_ptr<float>() : nullptr;
  a.bias = bias_desc(bias);
  a.batch = static_cast<int32_t>(B);
  a.heads = static_cast<int32_t>(H);
  a.seq_len = static_cast<int32_t>(N);
  a.head_dim = static_cast<int32_t>(D);
  a.dtype = code_of(q.scalar_type());
  a.summary_dtype = static_cast<int32_t>(summary_dtype);
  a.is_causal = causal ? 1 : 0;
  a.partition_len = static_cast<int32_t>(partition_len);
  a.q_chunk = static_cast<int32_t>(q_chunk);
  a.scale = 0.f;  // 1 / sqrt(head_dim)
  a.q_layout = layout_of(q);
  a.k_layout = layout_of(k);
  a.v_layout = layout_of(v);
  a.out_layout = layout_of(st.out);
  a.exact_row_max = 0;  // the state only feeds the backward (row_m + log2 row_z)
  elsa_fwd_plan plan;
  check(elsa_fwd_plan_get(&a, &plan), "elsa_fwd_plan_get");
  const at::Tensor ws = bytes(q, plan.workspace_bytes);
  a.workspace = ws.data_ptr();
  a.workspace_bytes = plan.workspace_bytes;
  check(elsa_fwd(&a, current_stream()), "elsa_fwd");
  return st;
}

// elsa_bwd into dq, dk, dv, then elsa_dbias when dbias_wanted; returns dbias (or undefined)
at::Tensor bwd_call(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& out,
                    const at::Tensor& dout_in, const at::Tensor& row_m, const at::Tensor& row_z, const at::Tensor& bias,
                    bool causal, const at::Tensor& dq, const at::Tensor& dk, const at::Tensor& dv, bool dbias_wanted) {
  const at::Tensor dout = operand(dout_in);
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  elsa_bwd_args b{};
  b.q = q.data_ptr();
  b.k = k.data_ptr();
  b.v = v.data_ptr();
  b.out = out.data_ptr();
  b.dout = dout.data_ptr();
  b.row_m = row_m.data_ptr<float>();
  b.row_z = row_z.data_ptr<float>();
  b.dq = dq.data_ptr();
  b.dk = dk.data_ptr();
  b.dv = dv.data_ptr();
  b.bias = bias_desc(bias);
  b.batch = static_cast<int32_t>(B);
  b.heads = static_cast<int32_t>(H);
  b.seq_len = static_cast<int32_t>(N);
  b.head_dim = static_cast<int32_t>(D);
  b.dtype = code_of(q.scalar_type());
  b.is_causal = causal ? 1 : 0;
  b.scale = 0.f;
  b.q_layout = layout_of(q);
  b.k_layout = layout_of(k);
  b.v_layout = layout_of(v);
  b.out_layout = layout_of(out);
  b.dout_layout = layout_of(dout);
  b.dq_layout = layout_of(dq);
  b.dk_layout = layout_of(dk);
  b.dv_layout = layout_of(dv);
  if (!bias.defined() || !dbias_wanted) {
    const size_t ws_bytes = elsa_bwd_workspace_bytes(&b);
    const at::Tensor ws = bytes(q, ws_bytes);
    b.workspace = ws.data_ptr();
    b.workspace_bytes = ws_bytes;
    check(elsa_bwd(&b, current_stream()), "elsa_bwd");
    return at::Tensor();
  }
  // dq, dk, dv and dbias in one call (dS from the dk/dv kernel)
  const int32_t bb = static_cast<int32_t>(bias.size(0)), bhd = static_cast<int32_t>(bias.size(1));
  at::Tensor d32 = at::empty({bb, bhd, N, N}, q.options().dtype(at::kFloat));
  const size_t need = elsa_bwd_dbias_workspace_bytes(&b, bb, bhd);
  const at::Tensor ws = bytes(q, need);
  b.workspace = ws.data_ptr();
  b.workspace_bytes = need;
  check(elsa_bwd_dbias(&b, d32.data_ptr<float>(), bb, bhd, current_stream()), "elsa_bwd_dbias");
  return d32.to(bias.scalar_type());
}

at::Tensor value_or_undefined(const c10::optional<at::Tensor>& t) { return t.has_value() ? *t : at::Tensor(); }

// The bias is an optional argument of both functions: an absent bias must not reach apply()
// as an undefined tensor, which autograd would treat as an input variable.

// q, k, v = qkv[:, :, 0..2] of a [B, N, 3, H, D] tensor; out as [B, N, H, D] memory; the
// gradient comes back as one [B, N, 3, H, D] tensor.
class QkvAttention : public torch::autograd::Function<QkvAttention> {
 public:
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& qkv, const c10::optional<at::Tensor>& bias_opt,
                            bool causal, int64_t summary_dtype, int64_t partition_len, int64_t q_chunk) {
    const c10::DeviceGuard guard(qkv.device());
    const at::Tensor bias = value_or_undefined(bias_opt);
    const auto t = unbind_qkv(qkv);
    FwdState st = fwd_call(t[0], t[1], t[2], bias, causal, summary_dtype, partition_len, q_chunk, true);
    ctx->save_for_backward({qkv, st.out, st.row_m, st.row_z, bias});
    ctx->saved_data["causal"] = causal;
    return st.out;
  }

  static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
    const auto sv = ctx->get_saved_variables();
    const c10::DeviceGuard guard(sv[0].device());
    const auto t = unbind_qkv(sv[0]);
    at::Tensor dqkv = at::empty(sv[0].sizes(), sv[0].options());
    const auto d = unbind_qkv(dqkv);
    const bool wants_dbias = sv[4].defined() && ctx->needs_input_grad(1);
    at::Tensor dbias = bwd_call(t[0], t[1], t[2], sv[1], grads[0], sv[2], sv[3], sv[4],
                                ctx->saved_data["causal"].toBool(), d[0], d[1], d[2], wants_dbias);
    return {dqkv, dbias, at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

// q, k, v as separate [B, H, N, D] tensors (any layout the ABI accepts); dense gradients.
class Attention : public torch::autograd::Function<Attention> {
 public:
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                            const c10::optional<at::Tensor>& bias_opt, bool causal, int64_t summary_dtype,
                            int64_t partition_len, int64_t q_chunk, bool out_bnhd) {
    const c10::DeviceGuard guard(q.device());
    const at::Tensor bias = value_or_undefined(bias_opt);
    FwdState st = fwd_call(q, k, v, bias, causal, summary_dtype, partition_len, q_chunk, out_bnhd);
    ctx->save_for_backward({q, k, v, st.out, st.row_m, st.row_z, bias});
    ctx->saved_data["causal"] = causal;
    return st.out;
  }

  static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
    const auto sv = ctx->get_saved_variables();
    const c10::DeviceGuard guard(sv[0].device());
    at::Tensor dq = at::empty(sv[0].sizes(), sv[0].options());
    at::Tensor dk = at::empty(sv[1].sizes(), sv[1].options());
    at::Tensor dv = at::empty(sv[2].sizes(), sv[2].options());
    const bool wants_dbias = sv[6].defined() && ctx->needs_input_grad(3);
    at::Tensor dbias = bwd_call(sv[0], sv[1], sv[2], sv[3], grads[0], sv[4], sv[5], sv[6],
                                ctx->saved_data["causal"].toBool(), dq, dk, dv, wants_dbias);
    return {dq, dk, dv, dbias, at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

void check_bias_arg(const c10::optional<at::Tensor>& bias, const at::Tensor& like) {
  TORCH_CHECK(!bias.has_value() || bias->dim() == 4, "bias must be a canonical [1|B,1|H,N,N] view");
  TORCH_CHECK(!bias.has_value() || bias->device() == like.device(), "bias must live on the same device as q");
}

at::Tensor qkv_attention_train(const at::Tensor& qkv, const c10::optional<at::Tensor>& bias, bool causal,
                               int64_t summary_dtype, int64_t partition_len, int64_t q_chunk) {
  TORCH_CHECK(qkv.dim() == 5 && qkv.size(2) == 3, "qkv must have shape [B,N,3,H,D]");
  TORCH_CHECK(qkv.is_contiguous(), "qkv must be contiguous");
  check_bias_arg(bias, qkv);
  return QkvAttention::apply(qkv, bias, causal, summary_dtype, partition_len, q_chunk);
}

at::Tensor attention_train(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                           const c10::optional<at::Tensor>& bias, bool causal, int64_t summary_dtype,
                           int64_t partition_len, int64_t q_chunk, bool out_bnhd) {
  TORCH_CHECK(q.dim() == 4 && q.sizes() == k.sizes() && q.sizes() == v.sizes(), "q, k, v must share one [B,H,N,D] shape");
  check_bias_arg(bias, q);
  return Attention::apply(q, k, v, bias, causal, summary_dtype, partition_len, q_chunk, out_bnhd);
}

// The inference forward (twopass_attention, reference attention.py:239-321) on operands the ABI
// reads in place: no row state, so the fold keeps the relaxed one.  Mirrors _elsa_forward in
// attention.py (the Python twin, used for inputs that need a padded copy), same arguments and bits.
at::Tensor attention_forward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                             const c10::optional<at::Tensor>& bias, bool causal, int64_t summary_dtype,
                             int64_t partition_len, int64_t q_chunk, bool out_bnhd) {
  TORCH_CHECK(q.dim() == 4 && q.sizes() == k.sizes() && q.sizes() == v.sizes(), "q, k, v must share one [B,H,N,D] shape");
  check_bias_arg(bias, q);
  const c10::DeviceGuard guard(q.device());
  return fwd_call(q, k, v, value_or_undefined(bias), causal, summary_dtype, partition_len, q_chunk, out_bnhd, false)
      .out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "C++ host side of the ELSA training (autograd) and inference calls";
  m.def("qkv_attention_train", &qkv_attention_train, "fused-qkv two-pass attention with recompute backward");
  m.def("attention_train", &attention_train, "two-pass attention on q, k, v with recompute backward");
  m.def("attention_forward", &attention_forward, "two-pass attention forward on q, k, v (inference)");
  m.def("current_stream", [] { return reinterpret_cast<int64_t>(current_stream()); },
        "raw handle of the stream the launches go to");
  m.def("abi_version", [] { return elsa_abi_version(); });
}
