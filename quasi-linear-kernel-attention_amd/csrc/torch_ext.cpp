// PyTorch C++ extension over libqlka.so's C ABI: the pybind module the reference's packages import as `_ext`
// (Weighted_Abs_Sum/csrc/binding.cpp:442-453, Weighted_Laplace_Sum/csrc/binding.cpp:102-105), with the same function
// names, arguments, checks and TORCH_CHECK messages, plus the autograd Functions of weighted_abs_sum(_full)
// (Weighted_Abs_Sum/weighted_abs_sum/ops.py:72-104) in C++, so that neither a call nor its backward runs Python.
//
// Host code only: every computation is a libqlka.so entry point (the gfx950 kernels). Outputs and workspaces come from
// torch's caching allocator on q's device, launches go on that device's current stream under a device guard.
#include <torch/extension.h>
#include <ATen/hip/HIPContext.h>
#include <c10/core/DeviceGuard.h>

#include <cstdint>
#include <tuple>

#include "qlka.h"

namespace {

using torch::Tensor;
using OptTensor = c10::optional<Tensor>;
using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

void check_rc(int rc) {
    if (rc != 0) {
        const char* msg = qlka_last_error();
        TORCH_CHECK(false, (msg && *msg) ? msg : "libqlka error");
    }
}

void* stream_of(const Tensor& t) { return (void*)at::hip::getCurrentHIPStream(t.device().index()).stream(); }

float* fptr(const Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }
float* fptr(const OptTensor& t) { return (t.has_value() && t->defined()) ? t->data_ptr<float>() : nullptr; }

struct Dims { int P, D, N, M, C; };

// check_qkv of Weighted_Abs_Sum/csrc/binding.cpp:69-84, same messages
Dims check_qkv(const Tensor& q, const Tensor& k, const Tensor& v) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "q, k, and v must be CUDA tensors");
    TORCH_CHECK(q.device() == k.device() && q.device() == v.device(), "q, k, and v must be on the same CUDA device");
    TORCH_CHECK(q.scalar_type() == at::kFloat && k.scalar_type() == at::kFloat && v.scalar_type() == at::kFloat,
                "q, k, and v must be float32");
    TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "q, k, and v must be 3D tensors");
    TORCH_CHECK(q.size(0) == k.size(0) && q.size(0) == v.size(0), "Batch size of q, k, and v must match");
    TORCH_CHECK(q.size(1) == k.size(1), "q and k must have same feature dimension");
    TORCH_CHECK(k.size(2) == v.size(1), "k and v must have same length");
    TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(), "q, k, and v must be contiguous");
    const int64_t P = q.size(0), D = q.size(1), N = k.size(2), C = v.size(2), M = q.size(2);
    TORCH_CHECK(M > 0 && N > 0 && D > 0, "N, M and D must be > 0");
    TORCH_CHECK(1 <= C && C <= 128, "C (v.size(2)) must be in [1, 128]");
    TORCH_CHECK(N <= 131072 && M <= 131072, "N and M must be <= 131072");
    TORCH_CHECK(P * D * std::max(N, M) <= INT32_MAX, "P*D*max(N,M) must fit int32 (cub sort offsets)");
    return {(int)P, (int)D, (int)N, (int)M, (int)C};
}

// the g / g_w / g_u checks (binding.cpp:251-262, 388-393)
void check_grad(const char* name, const Tensor& g, const Tensor& q, at::IntArrayRef shape) {
    TORCH_CHECK(g.is_cuda() && g.device() == q.device(), name, " must be on q's CUDA device");
    TORCH_CHECK(g.scalar_type() == at::kFloat, name, " must be float32");
    if (shape.size() == 3) {
        TORCH_CHECK(g.dim() == 3, name, " must be 3D");
        TORCH_CHECK(g.sizes() == shape, name, " must have shape (P, M, C)");
    } else {
        TORCH_CHECK(g.dim() == 2 && g.sizes() == shape, name, " must have shape (P, M)");
    }
    TORCH_CHECK(g.is_contiguous(), name, " must be contiguous");
}

void check_path(int64_t path) {
    TORCH_CHECK(-1 <= path && path <= 1, "path must be -1 (auto), 0 (global) or 1 (fused)");
}

Tensor workspace(size_t bytes, const Tensor& like) {
    return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

Tensor empty_f(at::IntArrayRef shape, const Tensor& like) { return at::empty(shape, like.options()); }

// ---- weighted_abs_sum

std::tuple<Tensor, OptTensor> abs_forward(const Tensor& q, const Tensor& k, const Tensor& v, int64_t path, bool full) {
    const Dims d = check_qkv(q, k, v);
    check_path(path);
    c10::DeviceGuard guard(q.device());
    Tensor out = empty_f({d.P, d.M, d.C}, q);
    OptTensor out_u;
    if (full) out_u = empty_f({d.P, d.M}, q);
    Tensor ws = workspace(qlka_abs_fwd_ws_bytes(d.P, d.D, d.N, d.M, d.C), q);
    check_rc(qlka_abs_fwd(fptr(q), fptr(k), fptr(v), fptr(out), fptr(out_u), d.P, d.D, d.N, d.M, d.C, (int)path,
                          ws.data_ptr(), (size_t)ws.numel(), stream_of(q)));
    return {out, out_u};
}

Tensor weighted_abs_sum_forward(const Tensor& q, const Tensor& k, const Tensor& v, int64_t path) {
    return std::get<0>(abs_forward(q, k, v, path, false));
}

std::tuple<Tensor, Tensor> weighted_abs_sum_full_forward(const Tensor& q, const Tensor& k, const Tensor& v,
                                                         int64_t path) {
    auto r = abs_forward(q, k, v, path, true);
    return {std::get<0>(r), *std::get<1>(r)};
}

// forward that also keeps the sorted k and q (with their permutations) when the backward at this shape walks
std::tuple<Tensor, OptTensor, std::vector<Tensor>> abs_forward_keep(const Tensor& q, const Tensor& k, const Tensor& v,
                                                                    int64_t path, bool full) {
    const Dims d = check_qkv(q, k, v);
    check_path(path);
    c10::DeviceGuard guard(q.device());
    Tensor out = empty_f({d.P, d.M, d.C}, q);
    OptTensor out_u;
    if (full) out_u = empty_f({d.P, d.M}, q);
    Tensor ws = workspace(qlka_abs_fwd_ws_bytes(d.P, d.D, d.N, d.M, d.C), q);
    std::vector<Tensor> srt;
    if (!qlka_abs_bwd_walks(d.P, d.N, d.M)) {
        check_rc(qlka_abs_fwd(fptr(q), fptr(k), fptr(v), fptr(out), fptr(out_u), d.P, d.D, d.N, d.M, d.C, (int)path,
                              ws.data_ptr(), (size_t)ws.numel(), stream_of(q)));
        return {out, out_u, srt};
    }
    const auto i32 = q.options().dtype(at::kInt);
    srt = {empty_f({d.P, d.D, d.N}, q), at::empty({d.P, d.D, d.N}, i32), empty_f({d.P, d.D, d.M}, q),
           at::empty({d.P, d.D, d.M}, i32)};
    // the walk's range states and bounds too, so that the backward's grad_q walk skips its range passes
    Tensor states = at::empty({(int64_t)qlka_abs_keep_state_bytes(d.P, d.D, d.N, d.M, d.C)},
                              q.options().dtype(at::kByte));
    int kept = 0;
    check_rc(qlka_abs_fwd_keep(fptr(q), fptr(k), fptr(v), fptr(out), fptr(out_u), d.P, d.D, d.N, d.M, d.C, (int)path,
                               fptr(srt[0]), (uint32_t*)srt[1].data_ptr<int32_t>(), fptr(srt[2]),
                               (uint32_t*)srt[3].data_ptr<int32_t>(), states.numel() ? states.data_ptr() : nullptr,
                               &kept, ws.data_ptr(), (size_t)ws.numel(), stream_of(q)));
    if (!kept) srt.clear();
    else if (kept & 2) srt.push_back(states);
    return {out, out_u, srt};
}

// The dense route's forward that keeps its kernel matrix A (P, M, (N + 3) & ~3) for the backward, and that backward
// (qlka_abs_fwd_dense_keep / qlka_abs_bwd_dense_kept): only where qlka_abs_dense_keep_bytes is nonzero.
std::tuple<Tensor, OptTensor, Tensor> abs_forward_dense_keep(const Tensor& q, const Tensor& k, const Tensor& v,
                                                             bool full) {
    const Dims d = check_qkv(q, k, v);
    c10::DeviceGuard guard(q.device());
    Tensor out = empty_f({d.P, d.M, d.C}, q);
    OptTensor out_u;
    if (full) out_u = empty_f({d.P, d.M}, q);
    Tensor A = empty_f({d.P, d.M, (d.N + 3) & ~int64_t(3)}, q);
    check_rc(qlka_abs_fwd_dense_keep(fptr(q), fptr(k), fptr(v), fptr(out), fptr(out_u), fptr(A), d.P, d.D, d.N, d.M,
                                     d.C, stream_of(q)));
    return {out, out_u, A};
}

std::tuple<Tensor, Tensor, Tensor> abs_backward_dense_kept(const Tensor& q, const Tensor& k, const Tensor& v,
                                                           const Tensor& g_w, const OptTensor& g_u, const Tensor& A) {
    const Dims d = check_qkv(q, k, v);
    check_grad("g_w", g_w, q, {d.P, d.M, d.C});
    if (g_u.has_value()) check_grad("g_u", *g_u, q, {d.P, d.M});
    TORCH_CHECK(A.sizes() == at::IntArrayRef({d.P, d.M, (d.N + 3) & ~int64_t(3)}) && A.is_contiguous(),
                "kept kernel matrix does not match q and k");
    c10::DeviceGuard guard(q.device());
    Tensor gq = empty_f({d.P, d.D, d.M}, q), gk = empty_f({d.P, d.D, d.N}, q), gv = empty_f({d.P, d.N, d.C}, q);
    check_rc(qlka_abs_bwd_dense_kept(fptr(q), fptr(k), fptr(v), fptr(g_w), fptr(g_u), fptr(gq), fptr(gk), fptr(gv),
                                     fptr(A), d.P, d.D, d.N, d.M, d.C, stream_of(q)));
    return {gq, gk, gv};
}

std::tuple<Tensor, Tensor, Tensor> abs_backward(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g_w,
                                                const OptTensor& g_u) {
    const Dims d = check_qkv(q, k, v);
    check_grad("g_w", g_w, q, {d.P, d.M, d.C});
    if (g_u.has_value()) check_grad("g_u", *g_u, q, {d.P, d.M});
    c10::DeviceGuard guard(q.device());
    Tensor gq = empty_f({d.P, d.D, d.M}, q), gk = empty_f({d.P, d.D, d.N}, q), gv = empty_f({d.P, d.N, d.C}, q);
    Tensor ws = workspace(qlka_abs_bwd_ws_bytes(d.P, d.D, d.N, d.M, d.C), q);
    check_rc(qlka_abs_bwd(fptr(q), fptr(k), fptr(v), fptr(g_w), fptr(g_u), fptr(gq), fptr(gk), fptr(gv), d.P, d.D,
                          d.N, d.M, d.C, ws.data_ptr(), (size_t)ws.numel(), stream_of(q)));
    return {gq, gk, gv};
}

std::tuple<Tensor, Tensor, Tensor> weighted_abs_sum_backward(const Tensor& q, const Tensor& k, const Tensor& v,
                                                             const Tensor& g_w) {
    return abs_backward(q, k, v, g_w, c10::nullopt);
}

std::tuple<Tensor, Tensor, Tensor> weighted_abs_sum_full_backward(const Tensor& q, const Tensor& k, const Tensor& v,
                                                                  const Tensor& g_w, const Tensor& g_u) {
    return abs_backward(q, k, v, g_w, g_u);
}

std::tuple<Tensor, Tensor, Tensor> abs_backward_sorted(const Tensor& q, const Tensor& k, const Tensor& v,
                                                       const Tensor& g_w, const OptTensor& g_u,
                                                       const std::vector<Tensor>& srt) {
    const Dims d = check_qkv(q, k, v);
    check_grad("g_w", g_w, q, {d.P, d.M, d.C});
    if (g_u.has_value()) check_grad("g_u", *g_u, q, {d.P, d.M});
    TORCH_CHECK((srt.size() == 4 || srt.size() == 5) && srt[0].sizes() == at::IntArrayRef({d.P, d.D, d.N}) &&
                    srt[1].sizes() == at::IntArrayRef({d.P, d.D, d.N}) &&
                    srt[2].sizes() == at::IntArrayRef({d.P, d.D, d.M}) &&
                    srt[3].sizes() == at::IntArrayRef({d.P, d.D, d.M}),
                "sorted arrays do not match q and k");
    const void* states = nullptr;
    if (srt.size() == 5) {
        TORCH_CHECK(srt[4].numel() == (int64_t)qlka_abs_keep_state_bytes(d.P, d.D, d.N, d.M, d.C) &&
                        srt[4].scalar_type() == at::kByte && srt[4].is_contiguous(),
                    "kept range states do not match q and k");
        states = srt[4].data_ptr();
    }
    c10::DeviceGuard guard(q.device());
    Tensor gq = empty_f({d.P, d.D, d.M}, q), gk = empty_f({d.P, d.D, d.N}, q), gv = empty_f({d.P, d.N, d.C}, q);
    Tensor ws = workspace(qlka_abs_bwd_ws_bytes(d.P, d.D, d.N, d.M, d.C), q);
    check_rc(qlka_abs_bwd_sorted(fptr(q), fptr(k), fptr(v), fptr(g_w), fptr(g_u), fptr(gq), fptr(gk), fptr(gv), d.P,
                                 d.D, d.N, d.M, d.C, fptr(srt[0]), (const uint32_t*)srt[1].data_ptr<int32_t>(),
                                 fptr(srt[2]), (const uint32_t*)srt[3].data_ptr<int32_t>(), states, ws.data_ptr(),
                                 (size_t)ws.numel(), stream_of(q)));
    return {gq, gk, gv};
}

Tensor weighted_sgn_sum_forward(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g) {
    const Dims d = check_qkv(q, k, v);
    check_grad("g", g, q, {d.P, d.M, d.C});
    c10::DeviceGuard guard(q.device());
    Tensor out = empty_f({d.P, d.D, d.M}, q);
    Tensor ws = workspace(qlka_sgn_fwd_ws_bytes(d.P, d.D, d.N, d.M, d.C), q);
    check_rc(qlka_sgn_fwd(fptr(q), fptr(k), fptr(v), fptr(g), fptr(out), d.P, d.D, d.N, d.M, d.C, ws.data_ptr(),
                          (size_t)ws.numel(), stream_of(q)));
    return out;
}

// ---- dense evaluation (the "keops" route)

std::tuple<Tensor, OptTensor> direct_forward(const Tensor& q, const Tensor& k, const Tensor& v, bool full) {
    const Dims d = check_qkv(q, k, v);
    c10::DeviceGuard guard(q.device());
    Tensor out = empty_f({d.P, d.M, d.C}, q);
    OptTensor out_u;
    if (full) out_u = empty_f({d.P, d.M}, q);
    check_rc(qlka_direct_fwd(0, fptr(q), fptr(k), fptr(v), fptr(out), fptr(out_u), d.P, d.D, d.N, d.M, d.C,
                             stream_of(q)));
    return {out, out_u};
}

std::tuple<Tensor, Tensor, Tensor> direct_backward(const Tensor& q, const Tensor& k, const Tensor& v,
                                                   const Tensor& g_w, const OptTensor& g_u, double tie) {
    const Dims d = check_qkv(q, k, v);
    check_grad("g_w", g_w, q, {d.P, d.M, d.C});
    if (g_u.has_value()) check_grad("g_u", *g_u, q, {d.P, d.M});
    c10::DeviceGuard guard(q.device());
    Tensor gq = empty_f({d.P, d.D, d.M}, q), gk = empty_f({d.P, d.D, d.N}, q), gv = empty_f({d.P, d.N, d.C}, q);
    check_rc(qlka_direct_bwd((float)tie, fptr(q), fptr(k), fptr(v), fptr(g_w), fptr(g_u), fptr(gq), fptr(gk),
                             fptr(gv), d.P, d.D, d.N, d.M, d.C, stream_of(q)));
    return {gq, gk, gv};
}

Tensor direct_sgn(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g, double tie) {
    const Dims d = check_qkv(q, k, v);
    check_grad("g", g, q, {d.P, d.M, d.C});
    c10::DeviceGuard guard(q.device());
    Tensor out = empty_f({d.P, d.D, d.M}, q);
    check_rc(qlka_direct_sgn((float)tie, fptr(q), fptr(k), fptr(v), fptr(g), fptr(out), d.P, d.D, d.N, d.M, d.C,
                             stream_of(q)));
    return out;
}

// ---- weighted_laplace_sum (Weighted_Laplace_Sum/csrc/binding.cpp:63-105, its messages)

std::tuple<Tensor, Tensor> weighted_laplace_sum_forward(const Tensor& q, const Tensor& k, const Tensor& v) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "q, k and v must be CUDA tensors");
    TORCH_CHECK(q.device() == k.device() && q.device() == v.device(), "q, k and v must be on one device");
    TORCH_CHECK(q.scalar_type() == at::kFloat && k.scalar_type() == at::kFloat && v.scalar_type() == at::kFloat,
                "q, k and v must be float32");
    TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "q, k and v must be 3D");
    TORCH_CHECK(q.size(0) == k.size(0) && q.size(0) == v.size(0), "batch size must match");
    TORCH_CHECK(q.size(1) == k.size(1), "q and k must have the same feature dimension");
    TORCH_CHECK(k.size(2) == v.size(1), "k and v must have the same length");
    TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(), "q, k and v must be contiguous");
    const int64_t P = q.size(0), D = q.size(1), N = k.size(2), C = v.size(2), M = q.size(2);
    TORCH_CHECK(M > 0 && N > 0 && D > 0, "N, M and D must be > 0");
    TORCH_CHECK(1 <= C && C <= 128, "C (v.size(2)) must be in [1, 128]");
    TORCH_CHECK(N <= 131072 && M <= 131072, "N and M must be <= 131072");
    TORCH_CHECK(P * D * std::max(N, M) <= INT32_MAX, "P*D*max(N,M) must fit int32 (cub sort offsets)");
    c10::DeviceGuard guard(q.device());
    Tensor out = empty_f({P, M, C}, q), out_u = empty_f({P, M}, q);
    Tensor ws = workspace(qlka_laplace_fwd_ws_bytes((int)P, (int)D, (int)N, (int)M, (int)C), q);
    check_rc(qlka_laplace_fwd(fptr(q), fptr(k), fptr(v), fptr(out), fptr(out_u), (int)P, (int)D, (int)N, (int)M,
                              (int)C, ws.data_ptr(), (size_t)ws.numel(), stream_of(q)));
    return {out, out_u};
}

// ---- autograd (Weighted_Abs_Sum/weighted_abs_sum/ops.py:72-104)
//
// path: -1 / 0 / 1 as the C entries take it, or DIRECT for the "keops" route (dense forward on contiguous copies,
// its gradient with sign(0) = 0). keep: keep the forward's sorts for the backward when a gradient is wanted.
constexpr int64_t DIRECT = 2;

struct AbsSumFn : public torch::autograd::Function<AbsSumFn> {
    static tensor_list forward(AutogradContext* ctx, Tensor q, Tensor k, Tensor v, int64_t path, bool full,
                               bool keep) {
        ctx->set_materialize_grads(false);
        ctx->saved_data["path"] = path;
        ctx->saved_data["full"] = full;
        std::vector<Tensor> srt;
        Tensor out;
        OptTensor out_u;
        bool dense_a = false;                 // srt holds the dense route's kernel matrix
        if (path == DIRECT) {
            q = q.contiguous();
            k = k.contiguous();
            v = v.contiguous();
            std::tie(out, out_u) = direct_forward(q, k, v, full);
        } else if (keep && q.dim() == 3 && k.dim() == 3 && v.dim() == 3 &&     // else check_qkv raises below
                   qlka_abs_dense_keep_bytes((int)q.size(0), (int)q.size(1), (int)k.size(2), (int)q.size(2),
                                             (int)v.size(2)) > 0) {
            Tensor A;
            std::tie(out, out_u, A) = abs_forward_dense_keep(q, k, v, full);
            srt = {A};
            dense_a = true;
        } else if (keep) {
            std::tie(out, out_u, srt) = abs_forward_keep(q, k, v, path, full);
        } else {
            std::tie(out, out_u) = abs_forward(q, k, v, path, full);
        }
        ctx->saved_data["sorted"] = !srt.empty() && !dense_a;
        ctx->saved_data["dense_a"] = dense_a;
        std::vector<Tensor> saved = {q, k, v};
        saved.insert(saved.end(), srt.begin(), srt.end());
        ctx->save_for_backward(saved);
        if (full) return {out, *out_u};
        return {out};
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        const auto saved = ctx->get_saved_variables();
        const Tensor& q = saved[0];
        const Tensor& k = saved[1];
        const Tensor& v = saved[2];
        const int64_t path = ctx->saved_data["path"].toInt();
        const bool full = ctx->saved_data["full"].toBool();
        Tensor g_w = grads[0];
        OptTensor g_u;
        if (full && grads.size() > 1 && grads[1].defined()) g_u = grads[1].contiguous();
        if (!g_w.defined()) g_w = at::zeros({q.size(0), q.size(2), v.size(2)}, q.options());
        g_w = g_w.contiguous();
        Tensor gq, gk, gv;
        if (path == DIRECT)
            std::tie(gq, gk, gv) = direct_backward(q, k, v, g_w, g_u, 0.0);
        else if (ctx->saved_data["dense_a"].toBool())
            std::tie(gq, gk, gv) = abs_backward_dense_kept(q, k, v, g_w, g_u, saved[3]);
        else if (ctx->saved_data["sorted"].toBool())
            std::tie(gq, gk, gv) = abs_backward_sorted(q, k, v, g_w, g_u,
                                                       std::vector<Tensor>(saved.begin() + 3, saved.end()));
        else
            std::tie(gq, gk, gv) = abs_backward(q, k, v, g_w, g_u);
        return {gq, gk, gv, Tensor(), Tensor(), Tensor()};
    }
};

std::vector<Tensor> abs_sum_autograd(const Tensor& q, const Tensor& k, const Tensor& v, int64_t path, bool full,
                                     bool keep) {
    return AbsSumFn::apply(q, k, v, path, full, keep);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    namespace py = pybind11;
    m.doc() = "weighted_abs_sum / weighted_laplace_sum entry points over libqlka.so (gfx950)";
    m.def("weighted_abs_sum_forward", &weighted_abs_sum_forward, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("path") = -1, "out[p,m,c] = sum_{n,d} |k[p,d,n] - q[p,d,m]| * v[p,n,c] (binding.cpp:229-233)");
    m.def("weighted_abs_sum_full_forward", &weighted_abs_sum_full_forward, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("path") = -1, "(out_w, out_u), out_u[p,m] = sum_{n,d} |k - q| (binding.cpp:235-239)");
    m.def("weighted_abs_sum_backward", &weighted_abs_sum_backward, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("g_w"), "(grad_q, grad_k, grad_v) of weighted_abs_sum (binding.cpp:370-374)");
    m.def("weighted_abs_sum_full_backward", &weighted_abs_sum_full_backward, py::arg("q"), py::arg("k"),
          py::arg("v"), py::arg("g_w"), py::arg("g_u"),
          "(grad_q, grad_k, grad_v) of weighted_abs_sum_full (binding.cpp:376-380)");
    m.def("weighted_sgn_sum_forward", &weighted_sgn_sum_forward, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("g"), "out[p,d,m] = sum_n sgn(k - q) dot(v[n], g[m]), a tie counted +1 (binding.cpp:383-439)");
    m.def("weighted_abs_sum_forward_keep", &abs_forward_keep, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("path"), py::arg("full"),
          "(out_w, out_u or None, [k_sorted, k_perm, q_sorted, q_perm (, range states)] or []): the forward that "
          "keeps its sorts (and, when it walked, its range states) when the backward at this shape walks "
          "(qlka_abs_fwd_keep)");
    m.def("weighted_abs_sum_backward_sorted", &abs_backward_sorted, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("g_w"), py::arg("g_u"), py::arg("srt"),
          "the backward over the sorts a weighted_abs_sum_forward_keep left (qlka_abs_bwd_sorted)");
    m.def("weighted_abs_sum_direct_forward", &direct_forward, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("full"), "dense (out_w, out_u or None) without a sort (qlka_direct_fwd)");
    m.def("weighted_abs_sum_direct_backward", &direct_backward, py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("g_w"), py::arg("g_u"), py::arg("tie"), "dense backward with sign(0) = tie (qlka_direct_bwd)");
    m.def("weighted_sgn_sum_direct", &direct_sgn, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("g"),
          py::arg("tie"), "dense weighted_sgn_sum with sign(0) = tie (qlka_direct_sgn)");
    m.def("weighted_laplace_sum_forward", &weighted_laplace_sum_forward, py::arg("q"), py::arg("k"), py::arg("v"),
          "(out_w, out_u) of the weighted Laplace sum (Weighted_Laplace_Sum/csrc/binding.cpp:102-105)");
    m.def("abs_sum_autograd", &abs_sum_autograd, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("path"),
          py::arg("full"), py::arg("keep"),
          "differentiable weighted_abs_sum (full=False: [out]) / weighted_abs_sum_full ([out_w, out_u]); path "
          "-1/0/1, or 2 for the dense route with sign(0) = 0 in the backward");
    m.attr("DIRECT") = DIRECT;
}
