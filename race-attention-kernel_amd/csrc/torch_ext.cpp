// torch_ext.cpp -- PyTorch-ROCm binding of the C ABI (include/race_mi355x.h).
//
//   forward(probsQ, probsK, V, causal, tile_tokens=0, kernel=0, want_state=False)
//       -> (out, state or None)
//   forward_debug(probsQ, probsK, V, causal, tile_tokens=0, kernel=0)
//       -> (out, records [N, tiles, rec], state [N, S*d+S], tile_tokens)
//   noncausal_backward(probsQ, probsK, V, dOut, state, need_q, need_k, need_v,
//                      tile_tokens=0) -> (dQ or None, dK or None, dV or None)
//   causal_backward(probsQ, probsK, V, dOut, need_q, need_k, need_v,
//                   tile_tokens=0, kernel=0) -> (dQ or None, dK or None, dV or None)
//   hash_probs(x, planes_T, L, K) -> [..., L, 2^K] bucket probabilities
//   select_tile_tokens(N, T, L, R, d, bf16, causal, tile_tokens=0, kernel=0) -> int
//   shape_supported(L, R, d) -> (supported, has_mfma)
//
// probsQ, probsK: [N, T, L, R] (or [N, T, S], read as L = 1, R = S) and V:
// [N, T, d], all float32 or all bfloat16, on one HIP device, contiguous,
// 16-byte aligned.  out has V's dtype; state is fp32.  The pattern follows the
// reference's binding (src/causal_v2/kernels/torch_binding.cpp:41-53 checks,
// :139-168 device guard, output and workspace allocation, current stream):
// TORCH_CHECK failures surface as RuntimeError.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>

#include <cstdint>
#include <tuple>
#include <vector>

#include "race_mi355x.h"

namespace {

constexpr int64_t kAlignment = 16;

void check_status(race_status st, const char* what) {
    TORCH_CHECK(st == RACE_SUCCESS, what, " failed: ", race_status_string(st), " (status ", st, ")");
}

void check_token_tensor(const at::Tensor& t, const char* name, const at::Tensor& like) {
    TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
    TORCH_CHECK(t.scalar_type() == at::kFloat || t.scalar_type() == at::kBFloat16, name,
                " must be float32 or bfloat16, got ", t.scalar_type());
    TORCH_CHECK(t.scalar_type() == like.scalar_type(), name, " dtype ", t.scalar_type(),
                " differs from probsQ ", like.scalar_type());
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
    TORCH_CHECK(t.device() == like.device(), name, " must be on the same device as probsQ");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(t.data_ptr()) % kAlignment == 0, name,
                " data must be 16-byte aligned (clone the tensor if it is a view)");
}

race_shape validate(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
    TORCH_CHECK(q.dim() == 4 || q.dim() == 3, "probsQ must be [N, T, L, R] or [N, T, S], got ",
                q.sizes());
    check_token_tensor(q, "probsQ", q);
    check_token_tensor(k, "probsK", q);
    check_token_tensor(v, "V", q);
    TORCH_CHECK(k.sizes() == q.sizes(), "probsK shape ", k.sizes(), " differs from probsQ ",
                q.sizes());
    TORCH_CHECK(v.dim() == 3, "V must be [N, T, d], got ", v.sizes());
    TORCH_CHECK(v.size(0) == q.size(0) && v.size(1) == q.size(1), "V ", v.sizes(),
                " does not match probsQ ", q.sizes(), " in N and T");
    race_shape sh;
    sh.num_streams = q.size(0);
    sh.seq_len = q.size(1);
    sh.num_tables = q.dim() == 4 ? static_cast<int32_t>(q.size(2)) : 1;
    sh.num_buckets = static_cast<int32_t>(q.dim() == 4 ? q.size(3) : q.size(2));
    sh.head_dim = static_cast<int32_t>(v.size(2));
    sh.dtype = q.scalar_type() == at::kBFloat16 ? RACE_BF16 : RACE_F32;
    int32_t supported = 0;
    check_status(race_shape_supported(&sh, &supported, nullptr), "race_shape_supported");
    TORCH_CHECK(supported, "unsupported shape: N=", sh.num_streams, " T=", sh.seq_len,
                " L=", sh.num_tables, " R=", sh.num_buckets, " d=", sh.head_dim,
                " (limits: N <= 65535, L*R <= 256, d <= 128)");
    return sh;
}

race_options make_options(int64_t tile_tokens, int64_t kernel) {
    TORCH_CHECK(tile_tokens >= 0 && tile_tokens % RACE_SUB_CHUNK_TOKENS == 0 &&
                    tile_tokens <= (int64_t(1) << 30),
                "tile_tokens must be 0 (automatic) or a positive multiple of ",
                RACE_SUB_CHUNK_TOKENS, ", got ", tile_tokens);
    TORCH_CHECK(kernel >= 0 && kernel <= 3,
                "kernel must be 0 (auto), 1 (valu), 2 (mfma) or 3 (mfma_wg)");
    race_options o;
    o.tile_tokens = static_cast<int32_t>(tile_tokens);
    o.kernel = static_cast<int32_t>(kernel);
    return o;
}

struct FwdResult {
    at::Tensor out, workspace, state;
    int64_t tiles = 0, rec = 0;
    int32_t tile = 0;
};

FwdResult run_forward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, bool causal,
                      int64_t tile_tokens, int64_t kernel, bool want_state) {
    const race_shape sh = validate(q, k, v);
    const race_options opts = make_options(tile_tokens, kernel);
    const c10::DeviceGuard guard(q.device());
    FwdResult r;
    r.out = at::empty_like(v);
    const int64_t S = int64_t(sh.num_tables) * sh.num_buckets;
    if (want_state)
        r.state = at::empty({sh.num_streams, S * sh.head_dim + S}, v.options().dtype(at::kFloat));
    size_t bytes = 0;
    check_status(race_fwd_workspace_bytes(&sh, causal, &opts, &bytes, &r.tiles, &r.rec),
                 "race_fwd_workspace_bytes");
    check_status(race_select_tile_tokens(&sh, causal, &opts, &r.tile), "race_select_tile_tokens");
    r.workspace = at::empty({static_cast<int64_t>((bytes + 3) / 4)}, v.options().dtype(at::kFloat));
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    check_status(race_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), r.out.data_ptr(),
                          want_state ? r.state.data_ptr<float>() : nullptr, &sh, causal, &opts,
                          r.workspace.data_ptr(), bytes, stream),
                 "race_fwd");
    return r;
}

std::tuple<at::Tensor, c10::optional<at::Tensor>> forward(const at::Tensor& q, const at::Tensor& k,
                                                          const at::Tensor& v, bool causal,
                                                          int64_t tile_tokens, int64_t kernel,
                                                          bool want_state) {
    FwdResult r = run_forward(q, k, v, causal, tile_tokens, kernel, want_state);
    if (want_state) return {r.out, r.state};
    return {r.out, c10::nullopt};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, int64_t> forward_debug(const at::Tensor& q,
                                                                      const at::Tensor& k,
                                                                      const at::Tensor& v,
                                                                      bool causal,
                                                                      int64_t tile_tokens,
                                                                      int64_t kernel) {
    FwdResult r = run_forward(q, k, v, causal, tile_tokens, kernel, true);
    const int64_t N = q.size(0);
    at::Tensor records;
    if (r.tiles > 0 && N > 0)
        records = r.workspace.narrow(0, 0, N * r.tiles * r.rec).view({N, r.tiles, r.rec});
    else
        records = at::zeros({N, 0, r.rec}, v.options().dtype(at::kFloat));
    return {r.out, records, r.state, r.tile};
}

std::tuple<c10::optional<at::Tensor>, c10::optional<at::Tensor>, c10::optional<at::Tensor>>
noncausal_backward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                   const at::Tensor& grad_out, const at::Tensor& state, bool need_q, bool need_k,
                   bool need_v, int64_t tile_tokens) {
    const race_shape sh = validate(q, k, v);
    check_token_tensor(grad_out, "dOut", q);
    TORCH_CHECK(grad_out.sizes() == v.sizes(), "dOut shape ", grad_out.sizes(), " differs from V ",
                v.sizes());
    const int64_t S = int64_t(sh.num_tables) * sh.num_buckets;
    TORCH_CHECK(state.is_cuda() && state.scalar_type() == at::kFloat && state.is_contiguous() &&
                    state.numel() == sh.num_streams * (S * sh.head_dim + S) &&
                    state.device() == q.device(),
                "state must be the forward's fp32 [N, S*d + S] state on the same device");
    const race_options opts = make_options(tile_tokens, RACE_KERNEL_AUTO);
    const c10::DeviceGuard guard(q.device());
    at::Tensor dq, dk, dv;
    if (need_q) dq = at::empty_like(q);
    if (need_k) dk = at::empty_like(k);
    if (need_v) dv = at::empty_like(v);
    size_t bytes = 0;
    check_status(race_noncausal_bwd_workspace_bytes(&sh, &opts, &bytes),
                 "race_noncausal_bwd_workspace_bytes");
    at::Tensor ws = at::empty({static_cast<int64_t>((bytes + 3) / 4)}, v.options().dtype(at::kFloat));
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    check_status(race_noncausal_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), grad_out.data_ptr(),
                                    state.data_ptr<float>(), need_q ? dq.data_ptr() : nullptr,
                                    need_k ? dk.data_ptr() : nullptr,
                                    need_v ? dv.data_ptr() : nullptr, &sh, &opts, ws.data_ptr(),
                                    bytes, stream),
                 "race_noncausal_bwd");
    auto opt = [](bool need, const at::Tensor& t) -> c10::optional<at::Tensor> {
        if (need) return t;
        return c10::nullopt;
    };
    return {opt(need_q, dq), opt(need_k, dk), opt(need_v, dv)};
}

std::tuple<c10::optional<at::Tensor>, c10::optional<at::Tensor>, c10::optional<at::Tensor>>
causal_backward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                const at::Tensor& grad_out, bool need_q, bool need_k, bool need_v,
                int64_t tile_tokens, int64_t kernel) {
    const race_shape sh = validate(q, k, v);
    check_token_tensor(grad_out, "dOut", q);
    TORCH_CHECK(grad_out.sizes() == v.sizes(), "dOut shape ", grad_out.sizes(), " differs from V ",
                v.sizes());
    const race_options opts = make_options(tile_tokens, kernel);
    const c10::DeviceGuard guard(q.device());
    at::Tensor dq, dk, dv;
    if (need_q) dq = at::empty_like(q);
    if (need_k) dk = at::empty_like(k);
    if (need_v) dv = at::empty_like(v);
    size_t bytes = 0;
    check_status(race_causal_bwd_workspace_bytes(&sh, &opts, &bytes),
                 "race_causal_bwd_workspace_bytes");
    at::Tensor ws = at::empty({static_cast<int64_t>((bytes + 3) / 4)}, v.options().dtype(at::kFloat));
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    check_status(race_causal_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), grad_out.data_ptr(),
                                 need_q ? dq.data_ptr() : nullptr, need_k ? dk.data_ptr() : nullptr,
                                 need_v ? dv.data_ptr() : nullptr, &sh, &opts, ws.data_ptr(), bytes,
                                 stream),
                 "race_causal_bwd");
    auto opt = [](bool need, const at::Tensor& t) -> c10::optional<at::Tensor> {
        if (need) return t;
        return c10::nullopt;
    };
    return {opt(need_q, dq), opt(need_k, dk), opt(need_v, dv)};
}

// [..., d_k] rows -> [..., L, 2^K] bucket probabilities (src/race_baseline.py:41-44).
at::Tensor hash_probs(const at::Tensor& x, const at::Tensor& planes_T, int64_t L, int64_t K) {
    TORCH_CHECK(x.is_cuda(), "x must be a GPU tensor");
    TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kBFloat16,
                "x must be float32 or bfloat16");
    TORCH_CHECK(x.is_contiguous() && reinterpret_cast<uintptr_t>(x.data_ptr()) % kAlignment == 0,
                "x must be contiguous and 16-byte aligned");
    TORCH_CHECK(x.dim() >= 1, "x must have a feature dimension");
    const int64_t dk = x.size(-1);
    TORCH_CHECK(planes_T.is_cuda() && planes_T.device() == x.device() &&
                    planes_T.scalar_type() == at::kFloat && planes_T.is_contiguous() &&
                    planes_T.dim() == 2 && planes_T.size(0) == dk && planes_T.size(1) == L * K,
                "planes_T must be a contiguous fp32 [d_k, L*K] tensor on x's device");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(planes_T.data_ptr()) % kAlignment == 0,
                "planes_T must be 16-byte aligned");
    const int64_t rows = x.numel() / dk;
    std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end() - 1);
    shape.push_back(L);
    shape.push_back(int64_t(1) << K);
    const c10::DeviceGuard guard(x.device());
    at::Tensor probs = at::empty(shape, x.options());
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    check_status(race_hash_probs(x.data_ptr(), planes_T.data_ptr<float>(), probs.data_ptr(), rows,
                                 static_cast<int32_t>(dk), static_cast<int32_t>(L),
                                 static_cast<int32_t>(K),
                                 x.scalar_type() == at::kBFloat16 ? RACE_BF16 : RACE_F32, stream),
                 "race_hash_probs");
    return probs;
}

int64_t select_tile_tokens(int64_t N, int64_t T, int64_t L, int64_t R, int64_t d, bool bf16,
                           bool causal, int64_t tile_tokens, int64_t kernel) {
    race_shape sh{N, T, static_cast<int32_t>(L), static_cast<int32_t>(R),
                  static_cast<int32_t>(d), bf16 ? RACE_BF16 : RACE_F32};
    const race_options opts = make_options(tile_tokens, kernel);
    int32_t tile = 0;
    check_status(race_select_tile_tokens(&sh, causal, &opts, &tile), "race_select_tile_tokens");
    return tile;
}

std::tuple<bool, bool> shape_supported(int64_t L, int64_t R, int64_t d) {
    race_shape sh{1, 1, static_cast<int32_t>(L), static_cast<int32_t>(R), static_cast<int32_t>(d),
                  RACE_F32};
    int32_t ok = 0, mfma = 0;
    check_status(race_shape_supported(&sh, &ok, &mfma), "race_shape_supported");
    return {ok != 0, mfma != 0};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    namespace py = pybind11;
    m.doc() = "Per-bucket RACE attention on MI355X (gfx950): PyTorch binding of librace_mi355x";
    m.def("forward", &forward, "race_fused_fwd(probsQ, probsK, V, causal) -> (out, state)",
          py::arg("probsQ"), py::arg("probsK"), py::arg("V"), py::arg("causal"),
          py::arg("tile_tokens") = 0, py::arg("kernel") = 0, py::arg("want_state") = false);
    m.def("forward_debug", &forward_debug,
          "Forward that also returns the scanned tile records, the state and the tile length",
          py::arg("probsQ"), py::arg("probsK"), py::arg("V"), py::arg("causal"),
          py::arg("tile_tokens") = 0, py::arg("kernel") = 0);
    m.def("noncausal_backward", &noncausal_backward, "Non-causal backward -> (dQ, dK, dV)",
          py::arg("probsQ"), py::arg("probsK"), py::arg("V"), py::arg("dOut"), py::arg("state"),
          py::arg("need_q") = true, py::arg("need_k") = true, py::arg("need_v") = true,
          py::arg("tile_tokens") = 0);
    m.def("causal_backward", &causal_backward, "Causal backward -> (dQ, dK, dV)",
          py::arg("probsQ"), py::arg("probsK"), py::arg("V"), py::arg("dOut"),
          py::arg("need_q") = true, py::arg("need_k") = true, py::arg("need_v") = true,
          py::arg("tile_tokens") = 0, py::arg("kernel") = 0);
    m.def("hash_probs", &hash_probs, "Bucket probabilities of token rows -> [..., L, 2^K]",
          py::arg("x"), py::arg("planes_T"), py::arg("L"), py::arg("K"));
    m.def("select_tile_tokens", &select_tile_tokens, "Tile length a forward would use",
          py::arg("N"), py::arg("T"), py::arg("L"), py::arg("R"), py::arg("d"),
          py::arg("bf16") = false, py::arg("causal") = true, py::arg("tile_tokens") = 0,
          py::arg("kernel") = 0);
    m.def("shape_supported", &shape_supported, "(supported, has_mfma) for (L, R, d)", py::arg("L"),
          py::arg("R"), py::arg("d"));
    m.def("abi_version", &race_abi_version, "ABI version of the loaded librace_mi355x");
}
