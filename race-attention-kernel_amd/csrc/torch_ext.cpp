// torch_ext.cpp -- PyTorch-ROCm binding of the C ABI (include/race_mi355x.h).
//
//   forward(probsQ, probsK, V, causal, tile_tokens=0, kernel=0, want_state=False)
//       -> (out, state or None)
//   forward_debug(probsQ, probsK, V, causal, tile_tokens=0, kernel=0)
//       -> (out, records [N, tiles, rec], state [N, S*d+S], tile_tokens)
//   forward_carry(probsQ, probsK, V, state, tile_tokens=0, kernel=0, inplace=False)
//       -> (out, state advanced over these tokens)
//   noncausal_backward(probsQ, probsK, V, dOut, state, need_q, need_k, need_v,
//                      tile_tokens=0) -> (dQ or None, dK or None, dV or None)
//   causal_backward(probsQ, probsK, V, dOut, need_q, need_k, need_v,
//                   tile_tokens=0, kernel=0) -> (dQ or None, dK or None, dV or None)
//   hash_probs(x, planes_T, L, K) -> [..., L, 2^K] bucket probabilities
//   select_tile_tokens(N, T, L, R, d, bf16, causal, tile_tokens=0, kernel=0) -> int
//   shape_supported(L, R, d) -> (supported, has_mfma)
//   alg1_forward(q, k, v, W, beta, tile_tokens=0, tensor_cores=False) -> out
//   alg1_forward_debug(q, k, v, W, beta, tile_tokens=0, tensor_cores=False)
//       -> (out, prefix_A, prefix_B, final_A, final_B, tile_tokens)
//   alg1_forward_carry(q, k, v, W, beta, state_A, state_B, tile_tokens=0, tensor_cores=False)
//       -> (out, final_A, final_B): continued from (state_A, state_B)
//   alg1_sub_chunk_tokens / alg1_select_tile_tokens / alg1_output_lds_bytes /
//   alg1_fits_on_device: the queries of the reference's causal v2 binding
//       (src/causal_v2/kernels/torch_binding.cpp:1-25)
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

race_options make_options(int64_t tile_tokens, int64_t kernel, bool allow_decode = false) {
    TORCH_CHECK(tile_tokens >= 0 && tile_tokens % RACE_SUB_CHUNK_TOKENS == 0 &&
                    tile_tokens <= (int64_t(1) << 30),
                "tile_tokens must be 0 (automatic) or a positive multiple of ",
                RACE_SUB_CHUNK_TOKENS, ", got ", tile_tokens);
    if (allow_decode) {
        TORCH_CHECK(kernel >= 0 && kernel <= RACE_KERNEL_DECODE,
                    "kernel must be 0 (auto), 1 (valu), 2 (mfma), 3 (mfma_wg) or 4 (decode)");
    } else {
        TORCH_CHECK(kernel >= 0 && kernel <= RACE_KERNEL_MFMA_WG,
                    "kernel must be 0 (auto), 1 (valu), 2 (mfma) or 3 (mfma_wg)");
    }
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

// Causal forward continued from a carried state [N, S*d + S] (B then A):
// returns (out, state after these tokens); with inplace the state is
// advanced in init_state itself and that tensor is returned.
std::tuple<at::Tensor, at::Tensor> forward_carry(const at::Tensor& q, const at::Tensor& k,
                                                 const at::Tensor& v, const at::Tensor& init_state,
                                                 int64_t tile_tokens, int64_t kernel, bool inplace) {
    const race_shape sh = validate(q, k, v);
    const race_options opts = make_options(tile_tokens, kernel, /*allow_decode=*/true);
    const int64_t S = int64_t(sh.num_tables) * sh.num_buckets;
    TORCH_CHECK(init_state.is_cuda() && init_state.scalar_type() == at::kFloat &&
                    init_state.is_contiguous() && init_state.device() == q.device(),
                "state must be a contiguous float32 tensor on the device of probsQ");
    TORCH_CHECK(init_state.dim() == 2 && init_state.size(0) == sh.num_streams &&
                    init_state.size(1) == S * sh.head_dim + S,
                "state must be [N, S*d + S] = [", sh.num_streams, ", ", S * sh.head_dim + S,
                "], got ", init_state.sizes());
    TORCH_CHECK(reinterpret_cast<uintptr_t>(init_state.data_ptr()) % kAlignment == 0,
                "state data must be 16-byte aligned");
    const c10::DeviceGuard guard(q.device());
    at::Tensor out = at::empty_like(v);
    at::Tensor state = inplace ? init_state : at::empty_like(init_state);
    size_t bytes = 0;
    check_status(race_fwd_carry_workspace_bytes(&sh, &opts, &bytes),
                 "race_fwd_carry_workspace_bytes");
    at::Tensor ws;
    if (bytes > 0)
        ws = at::empty({static_cast<int64_t>((bytes + 3) / 4)}, v.options().dtype(at::kFloat));
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    check_status(race_fwd_carry(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                init_state.data_ptr<float>(), state.data_ptr<float>(), &sh, &opts,
                                bytes > 0 ? ws.data_ptr() : nullptr, bytes, stream),
                 "race_fwd_carry");
    return {out, state};
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

// Causal forward for autograd: (out, scanned tile records [N, tiles, rec],
// tile length), the records being what the backward can start from.
std::tuple<at::Tensor, at::Tensor, int64_t> forward_with_records(const at::Tensor& q,
                                                                 const at::Tensor& k,
                                                                 const at::Tensor& v,
                                                                 int64_t tile_tokens,
                                                                 int64_t kernel) {
    FwdResult r = run_forward(q, k, v, true, tile_tokens, kernel, false);
    const int64_t N = q.size(0);
    at::Tensor records;
    if (r.tiles > 0 && N > 0)
        records = r.workspace.narrow(0, 0, N * r.tiles * r.rec).view({N, r.tiles, r.rec});
    else
        records = at::zeros({N, 0, r.rec}, v.options().dtype(at::kFloat));
    return {r.out, records, r.tile};
}

std::tuple<c10::optional<at::Tensor>, c10::optional<at::Tensor>, c10::optional<at::Tensor>>
causal_backward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                const at::Tensor& grad_out, bool need_q, bool need_k, bool need_v,
                int64_t tile_tokens, int64_t kernel, const c10::optional<at::Tensor>& fwd_records) {
    const race_shape sh = validate(q, k, v);
    check_token_tensor(grad_out, "dOut", q);
    TORCH_CHECK(grad_out.sizes() == v.sizes(), "dOut shape ", grad_out.sizes(), " differs from V ",
                v.sizes());
    const race_options opts = make_options(tile_tokens, kernel);
    if (fwd_records) {
        const at::Tensor& rec = *fwd_records;
        TORCH_CHECK(tile_tokens > 0, "saved forward records need the forward's tile length");
        TORCH_CHECK(rec.device() == q.device() && rec.scalar_type() == at::kFloat &&
                        rec.is_contiguous() && rec.dim() == 3 && rec.size(0) == q.size(0),
                    "fwd_records must be the forward's contiguous fp32 [N, tiles, rec] records");
        const int64_t tiles = (q.size(1) + tile_tokens - 1) / tile_tokens;
        TORCH_CHECK(rec.size(1) == tiles, "fwd_records has ", rec.size(1), " tiles, the tile length ",
                    tile_tokens, " gives ", tiles);
    }
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
    if (fwd_records && fwd_records->numel() > 0)
        check_status(race_causal_bwd_from_records(
                         q.data_ptr(), k.data_ptr(), v.data_ptr(), grad_out.data_ptr(),
                         fwd_records->data_ptr<float>(), need_q ? dq.data_ptr() : nullptr,
                         need_k ? dk.data_ptr() : nullptr, need_v ? dv.data_ptr() : nullptr, &sh,
                         &opts, ws.data_ptr(), bytes, stream),
                     "race_causal_bwd_from_records");
    else
        check_status(race_causal_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), grad_out.data_ptr(),
                                     need_q ? dq.data_ptr() : nullptr,
                                     need_k ? dk.data_ptr() : nullptr,
                                     need_v ? dv.data_ptr() : nullptr, &sh, &opts, ws.data_ptr(),
                                     bytes, stream),
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

// ---- Algorithm 1 with the hashing inside (race_alg1_*): the surface of the
// reference's causal v2 binding (src/causal_v2/kernels/torch_binding.cpp) ----

void check_alg1_token(const at::Tensor& t, const char* name, const at::Tensor& like) {
    TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
    TORCH_CHECK(t.scalar_type() == at::kBFloat16, name, " must be bfloat16, got ", t.scalar_type());
    TORCH_CHECK(t.dim() == 4, name, " must be [B, H, T, d], got ", t.sizes());
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
    TORCH_CHECK(t.sizes() == like.sizes(), name, " shape ", t.sizes(), " differs from q ", like.sizes());
    TORCH_CHECK(t.device() == like.device(), name, " must be on the same device as q");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(t.data_ptr()) % kAlignment == 0, name,
                " data must be 16-byte aligned (clone the tensor if it is a view)");
}

race_alg1_shape alg1_make_shape(int64_t batch_heads, int64_t seq_len, int64_t head_dim,
                                int64_t num_planes, int64_t num_tables) {
    TORCH_CHECK(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128, got ", head_dim);
    TORCH_CHECK(num_planes >= 1 && num_planes <= 5, "num_planes P must be in 1..5, got ", num_planes);
    TORCH_CHECK(num_tables >= 1 && num_tables <= 4, "num_tables L must be in 1..4, got ", num_tables);
    TORCH_CHECK(batch_heads >= 0 && batch_heads <= 65535, "batch * heads must be <= 65535, got ",
                batch_heads);
    TORCH_CHECK(seq_len >= 0 && seq_len <= int64_t(INT32_MAX) - RACE_ALG1_MAX_AUTO_TILE - 1,
                "sequence length out of range: ", seq_len);
    race_alg1_shape sh;
    sh.batch_heads = batch_heads;
    sh.seq_len = seq_len;
    sh.head_dim = static_cast<int32_t>(head_dim);
    sh.num_planes = static_cast<int32_t>(num_planes);
    sh.num_tables = static_cast<int32_t>(num_tables);
    return sh;
}

race_alg1_shape alg1_validate(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                              const at::Tensor& W, const at::Tensor& beta) {
    check_alg1_token(q, "q", q);
    check_alg1_token(k, "k", q);
    check_alg1_token(v, "v", q);
    TORCH_CHECK(W.device() == q.device(), "W must be on the same device as q");
    TORCH_CHECK(W.scalar_type() == at::kFloat, "W must be float32, got ", W.scalar_type());
    TORCH_CHECK(W.dim() == 3, "W must be [L, P, d], got ", W.sizes());
    TORCH_CHECK(W.is_contiguous(), "W must be contiguous");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(W.data_ptr()) % kAlignment == 0, "W must be 16-byte aligned");
    TORCH_CHECK(W.size(2) == q.size(3), "W head_dim ", W.size(2), " differs from q ", q.size(3));
    TORCH_CHECK(beta.numel() == 1, "beta must have exactly one element");
    TORCH_CHECK(at::isFloatingType(beta.scalar_type()), "beta must be a floating tensor");
    return alg1_make_shape(q.size(0) * q.size(1), q.size(2), q.size(3), W.size(1), W.size(0));
}

int32_t alg1_variant(bool tensor_cores) { return tensor_cores ? RACE_ALG1_BF16 : RACE_ALG1_FP32; }

int device_lds_limit() {
    int dev = 0, bytes = 0;
    TORCH_CHECK(hipGetDevice(&dev) == hipSuccess, "hipGetDevice failed");
    TORCH_CHECK(hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) ==
                    hipSuccess,
                "hipDeviceGetAttribute failed");
    return bytes;
}

void alg1_check_fits(const race_alg1_shape& sh, bool tensor_cores) {
    size_t bytes = 0;
    check_status(race_alg1_output_lds_bytes(&sh, alg1_variant(tensor_cores), &bytes),
                 "race_alg1_output_lds_bytes");
    const int limit = device_lds_limit();
    TORCH_CHECK(bytes <= size_t(limit), "the output pass needs ", bytes,
                " bytes of LDS per workgroup for d=", sh.head_dim, ", P=", sh.num_planes, ", L=",
                sh.num_tables, "; this GPU allows ", limit);
}

struct Alg1Result {
    at::Tensor out, workspace, final_state;
    int64_t tiles = 0, rec = 0;
    int32_t tile = 0;
};

Alg1Result alg1_run(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                    const at::Tensor& W, const at::Tensor& beta, int64_t tile_tokens,
                    bool tensor_cores, bool want_final, const at::Tensor* init = nullptr) {
    const race_alg1_shape sh = alg1_validate(q, k, v, W, beta);
    const c10::DeviceGuard guard(q.device());
    Alg1Result r;
    r.out = at::empty_like(q);
    if (sh.batch_heads == 0 || sh.seq_len == 0) return r;
    alg1_check_fits(sh, tensor_cores);
    TORCH_CHECK(tile_tokens == 0 || (tile_tokens > 0 && tile_tokens <= (int64_t(1) << 30) &&
                                     tile_tokens % RACE_ALG1_SUB_CHUNK_TOKENS == 0),
                "tile_tokens must be a positive multiple of ", RACE_ALG1_SUB_CHUNK_TOKENS, ", got ",
                tile_tokens);
    const int32_t variant = alg1_variant(tensor_cores);
    size_t bytes = 0;
    check_status(race_alg1_workspace_bytes(&sh, variant, static_cast<int32_t>(tile_tokens), &bytes,
                                           &r.tiles, &r.rec),
                 "race_alg1_workspace_bytes");
    r.tile = static_cast<int32_t>(tile_tokens);
    if (r.tile == 0) check_status(race_alg1_select_tile_tokens(&sh, variant, &r.tile), "race_alg1_select_tile_tokens");
    const auto fopt = q.options().dtype(at::kFloat);
    const at::Tensor beta_dev = beta.to(q.device(), at::kFloat).contiguous();
    r.workspace = at::empty({static_cast<int64_t>((bytes + 3) / 4)}, fopt);
    const int64_t S = int64_t(sh.num_tables) << sh.num_planes;
    if (want_final) r.final_state = at::empty({sh.batch_heads, S * sh.head_dim + S}, fopt);
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    float* fin = want_final ? r.final_state.data_ptr<float>() : nullptr;
    if (init) {
        check_status(race_alg1_fwd_carry(q.data_ptr(), k.data_ptr(), v.data_ptr(), W.data_ptr<float>(),
                                         beta_dev.data_ptr<float>(), r.out.data_ptr(),
                                         init->data_ptr<float>(), fin, &sh, r.tile, variant,
                                         r.workspace.data_ptr(), bytes, stream),
                     "race_alg1_fwd_carry");
    } else {
        check_status(race_alg1_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), W.data_ptr<float>(),
                                   beta_dev.data_ptr<float>(), r.out.data_ptr(), fin, &sh, r.tile,
                                   variant, r.workspace.data_ptr(), bytes, stream),
                     "race_alg1_fwd");
    }
    return r;
}

// Causal Algorithm 1 continued from a carried state (final_A [B, H, L, R] and
// final_B [B, H, L, R, D] fp32, as forward_debug returns them) -> (out,
// final_A, final_B) after these tokens.
std::tuple<at::Tensor, at::Tensor, at::Tensor> alg1_forward_carry(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& W,
    const at::Tensor& beta, const at::Tensor& state_A, const at::Tensor& state_B,
    int64_t tile_tokens, bool tensor_cores) {
    const race_alg1_shape sh = alg1_validate(q, k, v, W, beta);
    const int64_t B = q.size(0), H = q.size(1), D = q.size(3);
    const int64_t L = W.size(0), R = int64_t(1) << W.size(1), S = L * R;
    TORCH_CHECK(state_A.is_cuda() && state_A.scalar_type() == at::kFloat && state_A.device() == q.device() &&
                    state_A.sizes() == at::IntArrayRef({B, H, L, R}),
                "state_A must be a float32 [B, H, L, R] tensor on the device of q");
    TORCH_CHECK(state_B.is_cuda() && state_B.scalar_type() == at::kFloat && state_B.device() == q.device() &&
                    state_B.sizes() == at::IntArrayRef({B, H, L, R, D}),
                "state_B must be a float32 [B, H, L, R, D] tensor on the device of q");
    const c10::DeviceGuard guard(q.device());
    // The ABI's layout per stream: B [S][D] then A [S].
    const at::Tensor init = at::cat({state_B.reshape({B * H, S * D}), state_A.reshape({B * H, S})}, 1)
                                .contiguous();
    if (sh.batch_heads == 0 || sh.seq_len == 0)
        return {at::empty_like(q), state_A.clone(), state_B.clone()};
    Alg1Result r = alg1_run(q, k, v, W, beta, tile_tokens, tensor_cores, true, &init);
    const at::Tensor fin = r.final_state.view({B, H, S * D + S});
    return {r.out, fin.narrow(2, S * D, S).reshape({B, H, L, R}),
            fin.narrow(2, 0, S * D).reshape({B, H, L, R, D})};
}

at::Tensor alg1_forward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                        const at::Tensor& W, const at::Tensor& beta, int64_t tile_tokens,
                        bool tensor_cores) {
    return alg1_run(q, k, v, W, beta, tile_tokens, tensor_cores, false).out;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, int64_t> alg1_forward_debug(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& W,
    const at::Tensor& beta, int64_t tile_tokens, bool tensor_cores) {
    Alg1Result r = alg1_run(q, k, v, W, beta, tile_tokens, tensor_cores, true);
    const int64_t B = q.size(0), H = q.size(1), D = q.size(3);
    const int64_t L = W.size(0), R = int64_t(1) << W.size(1), S = L * R;
    const auto fopt = q.options().dtype(at::kFloat);
    if (!r.final_state.defined()) {
        return {r.out, at::zeros({B, H, 0, L, R}, fopt), at::zeros({B, H, 0, L, R, D}, fopt),
                at::zeros({B, H, L, R}, fopt), at::zeros({B, H, L, R, D}, fopt), 0};
    }
    // Records [BH][tiles][rec]: B [S][D] then A [S].
    const at::Tensor recs = r.workspace.narrow(0, 0, B * H * r.tiles * r.rec).view({B, H, r.tiles, r.rec});
    at::Tensor prefix_B = recs.narrow(3, 0, S * D).reshape({B, H, r.tiles, L, R, D}).clone();
    at::Tensor prefix_A = recs.narrow(3, S * D, S).reshape({B, H, r.tiles, L, R}).clone();
    const at::Tensor fin = r.final_state.view({B, H, S * D + S});
    at::Tensor final_B = fin.narrow(2, 0, S * D).reshape({B, H, L, R, D}).clone();
    at::Tensor final_A = fin.narrow(2, S * D, S).reshape({B, H, L, R}).clone();
    return {r.out, prefix_A, prefix_B, final_A, final_B, r.tile};
}

int64_t alg1_sub_chunk_tokens(int64_t head_dim, int64_t num_planes, bool tensor_cores) {
    alg1_make_shape(1, 1, head_dim, num_planes, 1);
    (void)tensor_cores;
    return RACE_ALG1_SUB_CHUNK_TOKENS;
}

int64_t alg1_select_tile_tokens(int64_t batch_heads, int64_t seq_len, int64_t head_dim,
                                int64_t num_planes, int64_t num_tables, bool tensor_cores) {
    const race_alg1_shape sh = alg1_make_shape(batch_heads, seq_len, head_dim, num_planes, num_tables);
    TORCH_CHECK(seq_len > 0 && batch_heads > 0, "empty shape has no tiles");
    alg1_check_fits(sh, tensor_cores);
    int32_t tile = 0;
    check_status(race_alg1_select_tile_tokens(&sh, alg1_variant(tensor_cores), &tile),
                 "race_alg1_select_tile_tokens");
    return tile;
}

int64_t alg1_output_lds_bytes(int64_t head_dim, int64_t num_planes, int64_t num_tables,
                              bool tensor_cores) {
    const race_alg1_shape sh = alg1_make_shape(1, 1, head_dim, num_planes, num_tables);
    size_t bytes = 0;
    check_status(race_alg1_output_lds_bytes(&sh, alg1_variant(tensor_cores), &bytes),
                 "race_alg1_output_lds_bytes");
    return static_cast<int64_t>(bytes);
}

bool alg1_fits_on_device(int64_t head_dim, int64_t num_planes, int64_t num_tables,
                         bool tensor_cores) {
    return alg1_output_lds_bytes(head_dim, num_planes, num_tables, tensor_cores) <= device_lds_limit();
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
    m.def("forward_carry", &forward_carry,
          "Causal forward continued from a carried state -> (out, state)", py::arg("probsQ"),
          py::arg("probsK"), py::arg("V"), py::arg("state"), py::arg("tile_tokens") = 0,
          py::arg("kernel") = 0, py::arg("inplace") = false);
    m.def("noncausal_backward", &noncausal_backward, "Non-causal backward -> (dQ, dK, dV)",
          py::arg("probsQ"), py::arg("probsK"), py::arg("V"), py::arg("dOut"), py::arg("state"),
          py::arg("need_q") = true, py::arg("need_k") = true, py::arg("need_v") = true,
          py::arg("tile_tokens") = 0);
    m.def("causal_backward", &causal_backward, "Causal backward -> (dQ, dK, dV)",
          py::arg("probsQ"), py::arg("probsK"), py::arg("V"), py::arg("dOut"),
          py::arg("need_q") = true, py::arg("need_k") = true, py::arg("need_v") = true,
          py::arg("tile_tokens") = 0, py::arg("kernel") = 0, py::arg("fwd_records") = py::none());
    m.def("forward_with_records", &forward_with_records,
          "Causal forward -> (out, scanned tile records, tile length) for the backward",
          py::arg("probsQ"), py::arg("probsK"), py::arg("V"), py::arg("tile_tokens") = 0,
          py::arg("kernel") = 0);
    m.def("hash_probs", &hash_probs, "Bucket probabilities of token rows -> [..., L, 2^K]",
          py::arg("x"), py::arg("planes_T"), py::arg("L"), py::arg("K"));
    m.def("select_tile_tokens", &select_tile_tokens, "Tile length a forward would use",
          py::arg("N"), py::arg("T"), py::arg("L"), py::arg("R"), py::arg("d"),
          py::arg("bf16") = false, py::arg("causal") = true, py::arg("tile_tokens") = 0,
          py::arg("kernel") = 0);
    m.def("shape_supported", &shape_supported, "(supported, has_mfma) for (L, R, d)", py::arg("L"),
          py::arg("R"), py::arg("d"));
    m.def("alg1_forward", &alg1_forward,
          "Causal Algorithm 1 with hashing: o = race_causal(q, k, v, W, beta)", py::arg("q"),
          py::arg("k"), py::arg("v"), py::arg("W"), py::arg("beta"), py::arg("tile_tokens") = 0,
          py::arg("tensor_cores") = false);
    m.def("alg1_forward_carry", &alg1_forward_carry,
          "alg1_forward continued from a carried state -> (out, final_A, final_B)", py::arg("q"),
          py::arg("k"), py::arg("v"), py::arg("W"), py::arg("beta"), py::arg("state_A"),
          py::arg("state_B"), py::arg("tile_tokens") = 0, py::arg("tensor_cores") = false);
    m.def("alg1_forward_debug", &alg1_forward_debug,
          "alg1_forward plus (prefix_A, prefix_B, final_A, final_B, tile_tokens)", py::arg("q"),
          py::arg("k"), py::arg("v"), py::arg("W"), py::arg("beta"), py::arg("tile_tokens") = 0,
          py::arg("tensor_cores") = false);
    m.def("alg1_sub_chunk_tokens", &alg1_sub_chunk_tokens, "Sub-chunk length C of the output pass",
          py::arg("head_dim"), py::arg("num_planes"), py::arg("tensor_cores") = false);
    m.def("alg1_select_tile_tokens", &alg1_select_tile_tokens,
          "Tile length the forward picks for this shape on the current device",
          py::arg("batch_heads"), py::arg("seq_len"), py::arg("head_dim"), py::arg("num_planes"),
          py::arg("num_tables"), py::arg("tensor_cores") = false);
    m.def("alg1_output_lds_bytes", &alg1_output_lds_bytes, "Dynamic LDS of the output pass in bytes",
          py::arg("head_dim"), py::arg("num_planes"), py::arg("num_tables"),
          py::arg("tensor_cores") = false);
    m.def("alg1_fits_on_device", &alg1_fits_on_device,
          "Whether the output pass fits this GPU's LDS", py::arg("head_dim"), py::arg("num_planes"),
          py::arg("num_tables"), py::arg("tensor_cores") = false);
    m.def("abi_version", &race_abi_version, "ABI version of the loaded librace_mi355x");
}
