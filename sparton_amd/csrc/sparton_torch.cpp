// Eager training ops of the SpartonHead path in C++ (libsparton_torch.so): the head, the MLM
// transform before it and the SPLADE loss after it, each with its autograd in C++, calling the
// C ABI of libsparton_hip.so (include/sparton.h). The modules (SpartonHead,
// SpartonMLMTransform, splade_loss) use these when torch.compile is not tracing, so that a
// training step dispatches no Python per op in the forward or the backward. The
// reference-named torch.library ops (sparton::fused_sparton_fwd/bwd, ...) are defined in
// Python, with their fake kernels; they compute the same things through the same C ABI and
// serve torch.compile and direct callers.
//
//   sparton_eager::head_train(hidden, weight, bias?, mask) -> reps
//       the training forward (reps, int32 argmax and fp32 reps from one kernel) whose backward
//       writes dH, dW, dbias rounded once to the parameters' dtype (sparton_kernel.py:643-707)
//   sparton_eager::head_encode(hidden, weight, bias?, mask) -> reps   (no argmax, no autograd)
//   sparton_eager::head_train_autocast(hidden, weight, bias?, mask, weight_c, bias_c?, pad)
//       -> reps; weight_c/bias_c are the compute-dtype copies of the fp32 masters weight/bias
//       (D zero-padded by pad); the backward writes fp32 gradients straight to the masters
//   sparton_eager::mlm_transform(x, weight, dense_bias, ln_weight, ln_bias, eps) -> y
//       LayerNorm(gelu(x W^T + b)) (training/model.py:14-40)
//   sparton_eager::splade_loss(q, d?, temperature, w_ce, w_l1, w_flops) -> out[6]
//       (total, CE, L1 q, L1 d, FLOPS q, FLOPS d)  (training/train.py:73-94, :164-197)
//
// The Python callers validate shapes and dtypes first (the same checks, and error types, as
// the torch.library ops); here only what the C ABI needs is enforced.
#include <ATen/ATen.h>
#include <ATen/hip/HIPContext.h>
#include <c10/core/DeviceGuard.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/library.h>

#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "../../include/sparton.h"

namespace {

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return SPARTON_F32;
    case at::kBFloat16: return SPARTON_BF16;
    case at::kHalf: return SPARTON_F16;
    default: TORCH_CHECK(false, "sparton: unsupported dtype ", t);
  }
}

// The forward's dtype: fp32 follows torch's float32 matmul precision ('high' and 'medium':
// the bf16 hi/lo split, SPARTON_F32_SPLIT; 'highest': exact fp32), as the reference's GEMM
// does under the 'high' it sets at import (sparton_kernel.py:14).
int fwd_dtype_code(at::ScalarType t) {
  const int code = dtype_code(t);
  if (t == at::kFloat &&
      at::globalContext().float32MatmulPrecision() != at::Float32MatmulPrecision::HIGHEST)
    return code | SPARTON_F32_SPLIT;
  return code;
}

int mask_code(at::ScalarType t) {
  switch (t) {
    case at::kLong: return SPARTON_MASK_I64;
    case at::kInt: return SPARTON_MASK_I32;
    case at::kBool:
    case at::kByte: return SPARTON_MASK_U8;
    case at::kFloat: return SPARTON_MASK_F32;
    case at::kBFloat16: return SPARTON_MASK_BF16;
    case at::kHalf: return SPARTON_MASK_F16;
    default: TORCH_CHECK(false, "sparton: unsupported mask dtype ", t);
  }
}

void check(int rc, const char* what) {
  TORCH_CHECK(rc == SPARTON_OK, "sparton: ", what, " failed with status ", rc, ": ", sparton_strerror(rc));
}

void* stream_of(const Tensor& t) { return at::hip::getCurrentHIPStream(t.device().index()).stream(); }

// Row-major, unit inner stride, 16-byte aligned base (what the C ABI requires); undefined stays.
Tensor dense(const Tensor& t) {
  if (!t.defined()) return t;
  Tensor c = t.contiguous();
  if (reinterpret_cast<uintptr_t>(c.data_ptr()) % 16 != 0) c = c.clone();
  return c;
}

const void* ptr(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }
void* mptr(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

Tensor workspace(size_t bytes, const Tensor& like) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// ---- the head --------------------------------------------------------------------------

struct FwdOut {
  Tensor reps, idx, reps32;
};

// sparton_fwd on dense tensors: reps in hidden's dtype, optionally the int32 argmax and fp32 reps.
FwdOut head_fwd(const Tensor& h, const Tensor& w, const Tensor& b, const Tensor& m, bool with_idx,
                bool with_f32) {
  const int64_t B = h.size(0), S = h.size(1), D = h.size(2), V = w.size(0);
  const int dt = fwd_dtype_code(h.scalar_type());
  FwdOut o;
  o.reps = at::empty({B, V}, h.options());
  if (with_idx) o.idx = at::empty({B, V}, h.options().dtype(at::kInt));
  if (with_f32) o.reps32 = at::empty({B, V}, h.options().dtype(at::kFloat));
  const size_t ws_bytes = sparton_fwd_workspace_bytes(B, S, D, V, dt);
  Tensor ws = workspace(ws_bytes, h);
  check(sparton_fwd(h.data_ptr(), w.data_ptr(), ptr(b), m.data_ptr(), mask_code(m.scalar_type()),
                    o.reps.data_ptr(), with_idx ? o.idx.data_ptr<int32_t>() : nullptr,
                    with_f32 ? o.reps32.data_ptr<float>() : nullptr, B, S, D, V, dt, ws.data_ptr(),
                    ws_bytes, stream_of(h)),
        "sparton_fwd");
  return o;
}

// sparton_bwd: gradients in `gdt` (fp32 or the inputs' dtype) from the fp32 reps.
std::tuple<Tensor, Tensor, Tensor> head_bwd(const Tensor& g, const Tensor& r32, const Tensor& idx,
                                            const Tensor& h, const Tensor& w, const Tensor& b,
                                            const Tensor& m, at::ScalarType gdt) {
  const int64_t B = h.size(0), S = h.size(1), D = h.size(2), V = w.size(0);
  const int dt = dtype_code(h.scalar_type());
  Tensor gd = dense(g.to(h.scalar_type()));
  Tensor dH = at::empty({B, S, D}, h.options().dtype(gdt));
  Tensor dW = at::empty({V, D}, h.options().dtype(gdt));
  Tensor db = at::empty({b.defined() ? V : 0}, h.options().dtype(gdt));
  const size_t ws_bytes = sparton_bwd_workspace_bytes(B, S, D, V);
  Tensor ws = workspace(ws_bytes, h);
  check(sparton_bwd(gd.data_ptr(), r32.data_ptr(), SPARTON_F32, idx.data_ptr<int32_t>(), m.data_ptr(),
                    mask_code(m.scalar_type()), h.data_ptr(), w.data_ptr(), dH.data_ptr(), dW.data_ptr(),
                    b.defined() ? db.data_ptr() : nullptr, dtype_code(gdt), ws.data_ptr(), ws_bytes, B, S,
                    D, V, dt, stream_of(h)),
        "sparton_bwd");
  return {dH, dW, db};
}

Tensor opt(const c10::optional<Tensor>& t) { return t.has_value() ? *t : Tensor(); }

// torch::autograd::Function::apply records the metadata of every tensor argument, which an
// undefined tensor does not have: an absent optional goes in as an empty placeholder and a
// flag, and is undefined again inside.
Tensor present(const c10::optional<Tensor>& t, const Tensor& like) {
  return t.has_value() ? *t : at::empty({0}, like.options());
}

// The forward's dispatch bodies: inference (no autograd) reps.
Tensor head_encode_cuda(const Tensor& hidden, const Tensor& weight, const c10::optional<Tensor>& bias,
                        const Tensor& mask) {
  c10::OptionalDeviceGuard guard(hidden.device());
  return head_fwd(dense(hidden), dense(weight), dense(opt(bias)), dense(mask), false, false).reps;
}

struct HeadTrainFn : public torch::autograd::Function<HeadTrainFn> {
  static Tensor forward(AutogradContext* ctx, const Tensor& hidden, const Tensor& weight,
                        const Tensor& bias_in, const Tensor& mask, bool has_bias) {
    at::AutoDispatchBelowADInplaceOrView below;
    c10::OptionalDeviceGuard guard(hidden.device());
    const Tensor bias = has_bias ? bias_in : Tensor();
    Tensor h = dense(hidden), w = dense(weight), b = dense(bias), m = dense(mask);
    FwdOut o = head_fwd(h, w, b, m, true, true);
    ctx->save_for_backward({o.reps32, o.idx, h, w, b, m});
    return o.reps;
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    auto s = ctx->get_saved_variables();
    const Tensor& b = s[4];
    if (!grads[0].defined()) return variable_list(5);
    c10::OptionalDeviceGuard guard(s[2].device());
    auto [dH, dW, db] = head_bwd(grads[0], s[0], s[1], s[2], s[3], b, s[5], s[2].scalar_type());
    return {dH, dW, b.defined() ? db : Tensor(), Tensor(), Tensor()};
  }
};

Tensor head_train_autograd(const Tensor& hidden, const Tensor& weight, const c10::optional<Tensor>& bias,
                           const Tensor& mask) {
  return HeadTrainFn::apply(hidden, weight, present(bias, hidden), mask, bias.has_value());
}

// Mixed precision: hidden and the masters weight/bias are fp32; weight_c/bias_c are their
// compute-dtype copies (D zero-padded by pad). The forward casts hidden the same way; the
// backward asks the kernels for fp32 gradients, which go to the masters unrounded.
struct HeadAutocastFn : public torch::autograd::Function<HeadAutocastFn> {
  static Tensor forward(AutogradContext* ctx, const Tensor& hidden, const Tensor& weight,
                        const Tensor& bias_in, const Tensor& mask, const Tensor& weight_c,
                        const Tensor& bias_c_in, int64_t pad, bool has_bias) {
    at::AutoDispatchBelowADInplaceOrView below;
    const Tensor bias = has_bias ? bias_in : Tensor();
    const Tensor bias_c = has_bias ? bias_c_in : Tensor();
    c10::OptionalDeviceGuard guard(hidden.device());
    Tensor h = hidden.to(weight_c.scalar_type());
    if (pad > 0) h = at::constant_pad_nd(h, {0, pad});
    h = dense(h);
    Tensor w = dense(weight_c), b = dense(bias_c), m = dense(mask);
    FwdOut o = head_fwd(h, w, b, m, true, true);
    ctx->save_for_backward({o.reps32, o.idx, h, w, b, m});
    ctx->saved_data["D"] = hidden.size(-1);
    ctx->saved_data["hidden_dtype"] = static_cast<int64_t>(hidden.scalar_type());
    ctx->saved_data["has_bias"] = bias.defined();
    return o.reps;
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    if (!grads[0].defined()) return variable_list(8);
    auto s = ctx->get_saved_variables();
    c10::OptionalDeviceGuard guard(s[2].device());
    auto [dH, dW, db] = head_bwd(grads[0], s[0], s[1], s[2], s[3], s[4], s[5], at::kFloat);
    const int64_t D = ctx->saved_data["D"].toInt();
    if (dH.size(-1) != D) {  // drop the zero padding columns
      dH = dH.narrow(-1, 0, D);
      dW = dW.narrow(-1, 0, D);
    }
    const auto hdt = static_cast<at::ScalarType>(ctx->saved_data["hidden_dtype"].toInt());
    return {dH.to(hdt), dW, ctx->saved_data["has_bias"].toBool() ? db : Tensor(),
            Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Tensor head_train_autocast_autograd(const Tensor& hidden, const Tensor& weight,
                                    const c10::optional<Tensor>& bias, const Tensor& mask,
                                    const Tensor& weight_c, const c10::optional<Tensor>& bias_c,
                                    int64_t pad) {
  TORCH_CHECK(bias.has_value() == bias_c.has_value(), "sparton: bias and its copy go together");
  return HeadAutocastFn::apply(hidden, weight, present(bias, hidden), mask, weight_c,
                               present(bias_c, weight_c), pad, bias.has_value());
}

// The CUDA-key bodies of the training ops, reached when no input needs a gradient (no
// autograd node is recorded): the reps alone.
Tensor head_train_cuda(const Tensor& hidden, const Tensor& weight, const c10::optional<Tensor>& bias,
                       const Tensor& mask) {
  return head_encode_cuda(hidden, weight, bias, mask);
}

Tensor head_train_autocast_cuda(const Tensor& hidden, const Tensor& weight,
                                const c10::optional<Tensor>& bias, const Tensor& mask,
                                const Tensor& weight_c, const c10::optional<Tensor>& bias_c, int64_t pad) {
  c10::OptionalDeviceGuard guard(hidden.device());
  Tensor h = hidden.to(weight_c.scalar_type());
  if (pad > 0) h = at::constant_pad_nd(h, {0, pad});
  return head_fwd(dense(h), dense(weight_c), dense(opt(bias_c)), dense(mask), false, false).reps;
}

// ---- cached hipBLASLt GEMMs (the transform's, 16-bit) ------------------------------------
//
// Column-major D[m x n] = op(A)[m x k] op(B)[k x n], fp32 accumulation, optionally a strided
// batch. torch's GEMM path asks hipBLASLt's heuristic for an algorithm on every call (~20 us of
// host time per GEMM); here the descriptors and the heuristic's first algorithm are made once
// per shape and device and kept, so a call is one hipblasLtMatmul. The library is the one
// torch loads (same soname), so the process holds one hipBLASLt.
struct GemmKey {
  int device, in_type, out_type, ta, tb, batch;
  int64_t m, n, k, lda, ldb, ldd, sa, sb, sd;
};
bool operator==(const GemmKey& x, const GemmKey& y) { return std::memcmp(&x, &y, sizeof(GemmKey)) == 0; }
struct GemmKeyHash {
  size_t operator()(const GemmKey& key) const {
    const unsigned char* p = reinterpret_cast<const unsigned char*>(&key);
    uint64_t h = 1469598103934665603ull;  // FNV-1a over the (zero-initialised) key bytes
    for (size_t i = 0; i < sizeof(GemmKey); ++i) h = (h ^ p[i]) * 1099511628211ull;
    return (size_t)h;
  }
};
struct GemmPlan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo;
  size_t ws = 0;
};
constexpr int kMaxGemmDevices = 64;
constexpr uint64_t kGemmMaxWorkspace = (uint64_t)32 << 20;
std::mutex g_lt_mu;
hipblasLtHandle_t g_lt[kMaxGemmDevices] = {};
std::unordered_map<GemmKey, GemmPlan, GemmKeyHash> g_plans;

void lt_check(hipblasStatus_t st, const char* what) {
  TORCH_CHECK(st == HIPBLAS_STATUS_SUCCESS, "sparton: hipBLASLt ", what, " failed (status ", (int)st, ")");
}

GemmKey gemm_key(int device, hipDataType in, hipDataType out, bool ta, bool tb, int64_t m, int64_t n,
                 int64_t k, int64_t lda, int64_t ldb, int64_t ldd, int batch = 1, int64_t sa = 0,
                 int64_t sb = 0, int64_t sd = 0) {
  GemmKey key;
  std::memset(&key, 0, sizeof(key));  // the padding bytes take part in == and the hash
  key.device = device;
  key.in_type = (int)in;
  key.out_type = (int)out;
  key.ta = ta;
  key.tb = tb;
  key.batch = batch;
  key.m = m;
  key.n = n;
  key.k = k;
  key.lda = lda;
  key.ldb = ldb;
  key.ldd = ldd;
  key.sa = sa;
  key.sb = sb;
  key.sd = sd;
  return key;
}

// Called with the key's device current. The returned reference stays valid: the map only grows.
const GemmPlan& gemm_plan(const GemmKey& key, hipblasLtHandle_t* handle) {
  TORCH_CHECK(key.device >= 0 && key.device < kMaxGemmDevices, "sparton: device index out of range");
  std::lock_guard<std::mutex> lock(g_lt_mu);
  if (g_lt[key.device] == nullptr) lt_check(hipblasLtCreate(&g_lt[key.device]), "handle creation");
  *handle = g_lt[key.device];
  auto it = g_plans.find(key);
  if (it != g_plans.end()) return it->second;
  GemmPlan p;
  lt_check(hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F), "descriptor");
  const hipblasOperation_t ta = key.ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const hipblasOperation_t tb = key.tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  lt_check(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)), "transA");
  lt_check(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)), "transB");
  const hipDataType in = (hipDataType)key.in_type, out = (hipDataType)key.out_type;
  lt_check(hipblasLtMatrixLayoutCreate(&p.a, in, key.ta ? key.k : key.m, key.ta ? key.m : key.k, key.lda), "layout A");
  lt_check(hipblasLtMatrixLayoutCreate(&p.b, in, key.tb ? key.n : key.k, key.tb ? key.k : key.n, key.ldb), "layout B");
  lt_check(hipblasLtMatrixLayoutCreate(&p.d, out, key.m, key.n, key.ldd), "layout D");
  if (key.batch > 1) {
    const int32_t bc = key.batch;
    const hipblasLtMatrixLayout_t lay[3] = {p.a, p.b, p.d};
    const int64_t str[3] = {key.sa, key.sb, key.sd};
    for (int i = 0; i < 3; ++i) {
      lt_check(hipblasLtMatrixLayoutSetAttribute(lay[i], HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)), "batch");
      lt_check(hipblasLtMatrixLayoutSetAttribute(lay[i], HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &str[i],
                                                 sizeof(str[i])), "batch stride");
    }
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  lt_check(hipblasLtMatmulPreferenceCreate(&pref), "preference");
  lt_check(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &kGemmMaxWorkspace,
                                                 sizeof(kGemmMaxWorkspace)), "workspace preference");
  hipblasLtMatmulHeuristicResult_t res[1];
  int got = 0;
  const hipblasStatus_t hs = hipblasLtMatmulAlgoGetHeuristic(*handle, p.op, p.a, p.b, p.d, p.d, pref, 1, res, &got);
  hipblasLtMatmulPreferenceDestroy(pref);
  lt_check(hs, "heuristic");
  TORCH_CHECK(got > 0, "sparton: hipBLASLt found no algorithm for a ", key.m, " x ", key.n, " x ", key.k, " GEMM");
  p.algo = res[0].algo;
  p.ws = res[0].workspaceSize;
  return g_plans.emplace(key, p).first->second;
}

void lt_gemm(const GemmKey& key, const void* A, const void* B, void* D, const Tensor& like) {
  hipblasLtHandle_t handle = nullptr;
  const GemmPlan& p = gemm_plan(key, &handle);
  Tensor ws = workspace(p.ws, like);
  const float alpha = 1.0f, beta = 0.0f;
  lt_check(hipblasLtMatmul(handle, p.op, &alpha, A, p.a, B, p.b, &beta, D, p.d, D, p.d, &p.algo,
                           p.ws ? ws.data_ptr() : nullptr, p.ws, (hipStream_t)stream_of(like)),
           "matmul");
}

hipDataType lt_type(at::ScalarType t) { return t == at::kBFloat16 ? HIP_R_16BF : HIP_R_16F; }
bool lt_gemm_ok(const Tensor& t) { return t.scalar_type() == at::kBFloat16 || t.scalar_type() == at::kHalf; }

// z[M, Dout] = x2[M, Din] W[Dout, Din]^T (column-major: z^T = op_T(W) x2^T).
Tensor lt_linear(const Tensor& x2, const Tensor& w) {
  const int64_t M = x2.size(0), Din = x2.size(1), Dout = w.size(0);
  Tensor z = at::empty({M, Dout}, x2.options());
  lt_gemm(gemm_key(x2.get_device(), lt_type(x2.scalar_type()), lt_type(x2.scalar_type()), true, false, Dout, M, Din,
                   Din, Din, Dout),
          w.data_ptr(), x2.data_ptr(), z.data_ptr(), x2);
  return z;
}

// dx[M, Din] = dz[M, Dout] W[Dout, Din] (column-major: dx^T = W^T dz^T, both as stored).
Tensor lt_dgrad(const Tensor& dz, const Tensor& w) {
  const int64_t M = dz.size(0), Dout = dz.size(1), Din = w.size(1);
  Tensor dx = at::empty({M, Din}, dz.options());
  lt_gemm(gemm_key(dz.get_device(), lt_type(dz.scalar_type()), lt_type(dz.scalar_type()), false, false, Din, M, Dout,
                   Din, Dout, Din),
          w.data_ptr(), dz.data_ptr(), dx.data_ptr(), dz);
  return dx;
}

// ---- the MLM transform -------------------------------------------------------------------

// Row chunks of the transform's batched weight-gradient GEMM, or 0 for one plain GEMM (the same
// rule as sparton_amd/transform.py's _wgrad_chunks).
int64_t wgrad_chunks(int64_t M, int64_t D, at::ScalarType dt) {
  if ((dt != at::kBFloat16 && dt != at::kHalf) || M < 2048 || D % 64 != 0) return 0;
  const int64_t C = M <= 4096 ? 4 : (M <= 16384 ? 8 : 16);
  return M % (C * 64) == 0 ? C : 0;
}

// dW = dz^T x2: row chunks transposed by HIP, one batched GEMM with fp32 outputs, the chunk
// products summed in order and rounded once by HIP (transform.py's _weight_grad).
// For 16-bit, the chunks go to hipBLASLt as one strided batch over row chunks of dz and x2 as
// they lie (dz transposed by the GEMM's op flag, so no transpose kernel): chunk i's fp32
// product is column-major (Din x Dout), i.e. row-major dW [Dout][Din].
Tensor transform_weight_grad(const Tensor& dz, const Tensor& x2, int64_t M, int64_t D) {
  const int64_t C = wgrad_chunks(M, D, dz.scalar_type());
  if (C == 0) {
    if (!lt_gemm_ok(dz)) return at::mm(dz.t(), x2);
    Tensor dw = at::empty({D, D}, dz.options());  // column-major dW^T = x2^T dz
    lt_gemm(gemm_key(dz.get_device(), lt_type(dz.scalar_type()), lt_type(dz.scalar_type()), false, true, D, D, M,
                     D, D, D),
            x2.data_ptr(), dz.data_ptr(), dw.data_ptr(), dz);
    return dw;
  }
  const int code = dtype_code(dz.scalar_type());
  void* st = stream_of(dz);
  const int64_t Mc = M / C;
  Tensor part = at::empty({C, D, D}, dz.options().dtype(at::kFloat));
  lt_gemm(gemm_key(dz.get_device(), lt_type(dz.scalar_type()), HIP_R_32F, false, true, D, D, Mc, D, D, D, (int)C,
                   Mc * D, Mc * D, D * D),
          x2.data_ptr(), dz.data_ptr(), part.data_ptr(), dz);
  Tensor dw = at::empty({D, D}, dz.options());
  check(sparton_transform_chunk_sum(part.data_ptr<float>(), dw.data_ptr(), C, D * D, code, st),
        "sparton_transform_chunk_sum");
  return dw;
}

struct TransformFn : public torch::autograd::Function<TransformFn> {
  static Tensor forward(AutogradContext* ctx, const Tensor& x, const Tensor& weight,
                        const Tensor& dense_bias, const Tensor& ln_weight, const Tensor& ln_bias,
                        double eps) {
    at::AutoDispatchBelowADInplaceOrView below;
    c10::OptionalDeviceGuard guard(x.device());
    const int64_t D = x.size(-1);
    Tensor x2 = x.reshape({-1, D});
    // hipBLASLt: cached plans for 16-bit, torch's F.linear otherwise
    Tensor z = lt_gemm_ok(x2) ? lt_linear(dense(x2), dense(weight)) : at::linear(x2, weight);
    const int64_t M = z.size(0);
    Tensor y = at::empty_like(z);
    Tensor mean = at::empty({M}, x.options().dtype(at::kFloat));
    Tensor rstd = at::empty({M}, x.options().dtype(at::kFloat));
    Tensor vb = dense_bias.contiguous(), vg = ln_weight.contiguous(), vt = ln_bias.contiguous();
    check(sparton_transform_fwd(z.data_ptr(), vb.data_ptr<float>(), vg.data_ptr<float>(),
                                vt.data_ptr<float>(), (float)eps, y.data_ptr(), mean.data_ptr<float>(),
                                rstd.data_ptr<float>(), M, D, dtype_code(x.scalar_type()), stream_of(x)),
          "sparton_transform_fwd");
    ctx->save_for_backward({x, weight, z, vb, vg, mean, rstd});
    return y.view(x.sizes());
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    if (!grads[0].defined()) return variable_list(6);
    auto s = ctx->get_saved_variables();
    const Tensor &x = s[0], &weight = s[1], &z = s[2], &vb = s[3], &vg = s[4], &mean = s[5], &rstd = s[6];
    c10::OptionalDeviceGuard guard(x.device());
    const int64_t D = x.size(-1);
    Tensor x2 = x.reshape({-1, D});
    const int64_t M = x2.size(0);
    Tensor dy2 = grads[0].reshape({-1, D}).to(x.scalar_type()).contiguous();
    Tensor dz = at::empty_like(z);
    Tensor dg = at::empty({D}, x.options().dtype(at::kFloat));
    Tensor dbt = at::empty_like(dg), dbd = at::empty_like(dg);
    const size_t ws_bytes = sparton_transform_workspace_bytes(M, D);
    Tensor ws = workspace(ws_bytes, x);
    check(sparton_transform_bwd(dy2.data_ptr(), z.data_ptr(), vb.data_ptr<float>(), vg.data_ptr<float>(),
                                mean.data_ptr<float>(), rstd.data_ptr<float>(), dz.data_ptr(),
                                dg.data_ptr<float>(), dbt.data_ptr<float>(), dbd.data_ptr<float>(),
                                ws.data_ptr(), ws_bytes, M, D, dtype_code(x.scalar_type()), stream_of(x)),
          "sparton_transform_bwd");
    Tensor dx = lt_gemm_ok(dz) ? lt_dgrad(dz, dense(weight)) : at::mm(dz, weight);
    Tensor dw = transform_weight_grad(dz, lt_gemm_ok(dz) ? dense(x2) : x2, M, D);
    return {dx.view(x.sizes()), dw, dbd, dg, dbt, Tensor()};
  }
};

Tensor transform_autograd(const Tensor& x, const Tensor& weight, const Tensor& dense_bias,
                          const Tensor& ln_weight, const Tensor& ln_bias, double eps) {
  return TransformFn::apply(x, weight, dense_bias, ln_weight, ln_bias, eps);
}

Tensor transform_cuda(const Tensor& x, const Tensor& weight, const Tensor& dense_bias,
                      const Tensor& ln_weight, const Tensor& ln_bias, double eps) {
  c10::OptionalDeviceGuard guard(x.device());
  const int64_t D = x.size(-1);
  Tensor x2 = x.reshape({-1, D});
  Tensor z = lt_gemm_ok(x2) ? lt_linear(dense(x2), dense(weight)) : at::linear(x2, weight);
  const int64_t M = z.size(0);
  Tensor y = at::empty_like(z);
  Tensor mean = at::empty({M}, x.options().dtype(at::kFloat)), rstd = at::empty_like(mean);
  Tensor vb = dense_bias.contiguous(), vg = ln_weight.contiguous(), vt = ln_bias.contiguous();
  check(sparton_transform_fwd(z.data_ptr(), vb.data_ptr<float>(), vg.data_ptr<float>(),
                              vt.data_ptr<float>(), (float)eps, y.data_ptr(), mean.data_ptr<float>(),
                              rstd.data_ptr<float>(), M, D, dtype_code(x.scalar_type()), stream_of(x)),
        "sparton_transform_fwd");
  return y.view(x.sizes());
}

// ---- the SPLADE loss ----------------------------------------------------------------------

std::tuple<Tensor, Tensor> loss_fwd(const Tensor& q, const Tensor& d, double T, double w_ce,
                                    double w_l1, double w_flops) {
  const int64_t Bq = q.size(0), V = q.size(1), Bd = d.defined() ? d.size(0) : 0;
  Tensor out = at::empty({6}, q.options().dtype(at::kFloat));
  Tensor probs = at::empty({Bq, Bd}, q.options().dtype(at::kFloat));
  const size_t ws_bytes = sparton_loss_workspace_bytes(Bq, Bd, V);
  Tensor ws = workspace(ws_bytes, q);
  check(sparton_loss_fwd(q.data_ptr(), ptr(d), Bq, Bd, V, (float)T, (float)w_ce, (float)w_l1,
                         (float)w_flops, out.data_ptr<float>(), Bd ? probs.data_ptr<float>() : nullptr,
                         ws.data_ptr(), ws_bytes, dtype_code(q.scalar_type()), stream_of(q)),
        "sparton_loss_fwd");
  return {out, probs};
}

// The six terms (total, CE, L1(q), L1(d), FL(q), FL(d)) as separate scalars (views of the
// kernel's one output buffer), so that a caller backpropagating some of them (usually
// `total`) hands the backward only those gradients: the others stay undefined (no
// materialised zeros, no stack of six) and reach the kernel as NULL pointers.
using Loss6 = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>;
Loss6 split6(const Tensor& out) {
  return {out.select(0, 0), out.select(0, 1), out.select(0, 2), out.select(0, 3), out.select(0, 4),
          out.select(0, 5)};
}

struct LossFn : public torch::autograd::Function<LossFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& q_in, const Tensor& d_in, bool has_d,
                               double T, double w_ce, double w_l1, double w_flops) {
    at::AutoDispatchBelowADInplaceOrView below;
    c10::OptionalDeviceGuard guard(q_in.device());
    Tensor q = q_in.contiguous(), d = has_d ? d_in.contiguous() : Tensor();
    auto [out, probs] = loss_fwd(q, d, T, w_ce, w_l1, w_flops);
    ctx->save_for_backward({q, d, probs});
    ctx->saved_data["w_ce"] = w_ce;
    ctx->saved_data["w_l1"] = w_l1;
    ctx->saved_data["w_flops"] = w_flops;
    ctx->set_materialize_grads(false);
    auto t = split6(out);
    return {std::get<0>(t), std::get<1>(t), std::get<2>(t), std::get<3>(t), std::get<4>(t), std::get<5>(t)};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const float* gp[6];
    std::vector<Tensor> keep;
    bool any = false;
    for (int k = 0; k < 6; ++k) {
      gp[k] = nullptr;
      if (grads[k].defined()) {
        keep.push_back(grads[k].to(at::kFloat).contiguous());
        gp[k] = keep.back().data_ptr<float>();
        any = true;
      }
    }
    if (!any) return variable_list(7);
    auto s = ctx->get_saved_variables();
    const Tensor &q = s[0], &d = s[1], &probs = s[2];
    c10::OptionalDeviceGuard guard(q.device());
    const int64_t Bq = q.size(0), V = q.size(1), Bd = d.defined() ? d.size(0) : 0;
    Tensor dq = at::empty_like(q);
    Tensor dd = d.defined() ? at::empty_like(d) : Tensor();
    check(sparton_loss_bwd_terms(q.data_ptr(), ptr(d), Bd ? probs.data_ptr<float>() : nullptr, gp, Bq, Bd,
                                 V, (float)ctx->saved_data["w_ce"].toDouble(),
                                 (float)ctx->saved_data["w_l1"].toDouble(),
                                 (float)ctx->saved_data["w_flops"].toDouble(), dq.data_ptr(), mptr(dd),
                                 dtype_code(q.scalar_type()), stream_of(q)),
          "sparton_loss_bwd_terms");
    return {dq, dd, Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Loss6 loss_autograd(const Tensor& q, const c10::optional<Tensor>& d, double T, double w_ce, double w_l1,
                    double w_flops) {
  auto o = LossFn::apply(q, present(d, q), d.has_value(), T, w_ce, w_l1, w_flops);
  return {o[0], o[1], o[2], o[3], o[4], o[5]};
}

Loss6 loss_cuda(const Tensor& q, const c10::optional<Tensor>& d, double T, double w_ce, double w_l1,
                double w_flops) {
  c10::OptionalDeviceGuard guard(q.device());
  Tensor dd = d.has_value() ? d->contiguous() : Tensor();
  return split6(std::get<0>(loss_fwd(q.contiguous(), dd, T, w_ce, w_l1, w_flops)));
}

// CPU tensors: the same refusal as the reference's `assert hidden.is_cuda`
// (sparton_kernel.py:650), as a RuntimeError.
[[noreturn]] void cpu_refused(const char* op) {
  TORCH_CHECK(false, op, " only supports ROCm/HIP device tensors (got a CPU tensor)");
}

}  // namespace

TORCH_LIBRARY(sparton_eager, m) {
  m.def("head_train(Tensor hidden, Tensor weight, Tensor? bias, Tensor mask) -> Tensor");
  m.def("head_encode(Tensor hidden, Tensor weight, Tensor? bias, Tensor mask) -> Tensor");
  m.def("head_train_autocast(Tensor hidden, Tensor weight, Tensor? bias, Tensor mask, "
        "Tensor weight_c, Tensor? bias_c, int pad) -> Tensor");
  m.def("mlm_transform(Tensor x, Tensor weight, Tensor dense_bias, Tensor ln_weight, "
        "Tensor ln_bias, float eps) -> Tensor");
  m.def("splade_loss(Tensor q, Tensor? d, float temperature, float w_ce, float w_l1, "
        "float w_flops) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(sparton_eager, CUDA, m) {
  m.impl("head_train", &head_train_cuda);
  m.impl("head_encode", &head_encode_cuda);
  m.impl("head_train_autocast", &head_train_autocast_cuda);
  m.impl("mlm_transform", &transform_cuda);
  m.impl("splade_loss", &loss_cuda);
}

TORCH_LIBRARY_IMPL(sparton_eager, AutogradCUDA, m) {
  m.impl("head_train", &head_train_autograd);
  m.impl("head_train_autocast", &head_train_autocast_autograd);
  m.impl("mlm_transform", &transform_autograd);
  m.impl("splade_loss", &loss_autograd);
}

TORCH_LIBRARY_IMPL(sparton_eager, CPU, m) {
  m.impl("head_train", [](const Tensor&, const Tensor&, const c10::optional<Tensor>&, const Tensor&) -> Tensor {
    cpu_refused("sparton_eager::head_train");
  });
  m.impl("head_encode", [](const Tensor&, const Tensor&, const c10::optional<Tensor>&, const Tensor&) -> Tensor {
    cpu_refused("sparton_eager::head_encode");
  });
  m.impl("head_train_autocast",
         [](const Tensor&, const Tensor&, const c10::optional<Tensor>&, const Tensor&, const Tensor&,
            const c10::optional<Tensor>&, int64_t) -> Tensor { cpu_refused("sparton_eager::head_train_autocast"); });
  m.impl("mlm_transform", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                             double) -> Tensor { cpu_refused("sparton_eager::mlm_transform"); });
  m.impl("splade_loss", [](const Tensor&, const c10::optional<Tensor>&, double, double, double,
                           double) -> Loss6 { cpu_refused("sparton_eager::splade_loss"); });
}
