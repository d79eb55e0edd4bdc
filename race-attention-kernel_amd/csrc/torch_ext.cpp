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
//   hash_probs_backward(x, planes_T, dprobs, L, K) -> dx
//   hashed_forward(K, Q, V, planes, L, tile_tokens=0, want_records=False, want_state=False)
//       -> (out, records or None, state or None, tile_tokens): the causal op
//       with the hashing inside (race_hashed_fwd)
//   hashed_supported(L, K, d) -> bool
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
// 16-byte aligned.  out has V's dtype; state is fp32.  As the reference's
// binding does (src/causal_v2/kernels/torch_binding.cpp:139-168), every entry
// point checks its arguments on the host, allocates the outputs and the
// workspace itself and launches on PyTorch's current stream under a device
// guard; a rejected argument raises RuntimeError naming the entry point, the
// argument and the rule it broke.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>

#include <algorithm>
#include <cstdint>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "race_mi355x.h"

namespace {

// ---- argument checking ----------------------------------------------------
// The kernels address token rows through 16-byte buffer loads and stores, so
// every tensor handed to the library is dense row-major storage on the GPU
// with a 16-byte aligned base.  ArgCheck walks an entry point's arguments,
// keeps the first requirement that fails and raises it as one RuntimeError
// naming the entry point, the argument and the requirement.
class ArgCheck {
  public:
    explicit ArgCheck(const char* entry) : entry_(entry) {}

    // Dense, 16-byte aligned storage on a GPU.
    ArgCheck& on_gpu(const char* name, const at::Tensor& t) {
        if (!t.is_cuda())
            fail(name, "lives on the CPU; the library reads it on the GPU");
        else if (!t.is_contiguous())
            fail(name, "is a strided view; pass a contiguous tensor");
        else if (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 != 0)
            fail(name, "starts at an address that is not a multiple of 16 bytes; pass a fresh copy");
        return *this;
    }
    // One of the accepted element types.
    ArgCheck& dtype_is(const char* name, const at::Tensor& t, bool allow_f32) {
        const auto st = t.scalar_type();
        if (st != at::kBFloat16 && !(allow_f32 && st == at::kFloat))
            fail(name, allow_f32 ? "holds neither float32 nor bfloat16 elements"
                                 : "holds elements other than bfloat16");
        return *this;
    }
    // Same element type and device as the reference argument.
    ArgCheck& matches(const char* name, const at::Tensor& t, const char* ref_name,
                      const at::Tensor& ref) {
        if (t.scalar_type() != ref.scalar_type()) fail(name, std::string("has another dtype than ") + ref_name);
        if (t.device() != ref.device()) fail(name, std::string("lives on another device than ") + ref_name);
        return *this;
    }
    // A free-form requirement.
    ArgCheck& require(bool ok, const char* name, const std::string& what) {
        if (!ok) fail(name, what);
        return *this;
    }
    void raise() const {
        TORCH_CHECK(reason_.empty(), entry_, ": ", reason_);
    }

  private:
    void fail(const char* name, const std::string& what) {
        if (reason_.empty()) reason_ = std::string(name) + " " + what;
    }
    const char* entry_;
    std::string reason_;
};

std::string dims(const at::Tensor& t) {
    std::ostringstream s;
    s << t.sizes();
    return s.str();
}

void check_status(race_status st, const char* what) {
    TORCH_CHECK(st == RACE_SUCCESS, what, " failed: ", race_status_string(st), " (status ", st, ")");
}

// The per-bucket op's three token tensors: probs [N, T, L, R] (or [N, T, S])
// and V [N, T, d], all float32 or all bfloat16 on one device.
race_shape validate(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                    const char* entry = "race_fused_fwd") {
    ArgCheck c(entry);
    c.require(q.dim() == 3 || q.dim() == 4, "probsQ", "has shape " + dims(q) + ", not [N, T, L, R] or [N, T, S]")
        .on_gpu("probsQ", q).dtype_is("probsQ", q, true)
        .on_gpu("probsK", k).matches("probsK", k, "probsQ", q)
        .require(k.sizes() == q.sizes(), "probsK", "has shape " + dims(k) + ", probsQ " + dims(q))
        .on_gpu("V", v).matches("V", v, "probsQ", q)
        .require(v.dim() == 3 && v.size(0) == q.size(0) && v.size(1) == q.size(1), "V",
                 "has shape " + dims(v) + ", not [N, T, d] with probsQ's N and T");
    c.raise();
    race_shape sh;
    sh.num_streams = q.size(0);
    sh.seq_len = q.size(1);
    sh.num_tables = q.dim() == 4 ? static_cast<int32_t>(q.size(2)) : 1;
    sh.num_buckets = static_cast<int32_t>(q.size(q.dim() - 1));
    sh.head_dim = static_cast<int32_t>(v.size(2));
    sh.dtype = q.scalar_type() == at::kBFloat16 ? RACE_BF16 : RACE_F32;
    int32_t supported = 0;
    check_status(race_shape_supported(&sh, &supported, nullptr), "race_shape_supported");
    TORCH_CHECK(supported, entry, ": no kernel takes N=", sh.num_streams, ", T=", sh.seq_len,
                ", S=L*R=", int64_t(sh.num_tables) * sh.num_buckets, ", d=", sh.head_dim,
                "; the library covers N <= 65535 streams, S <= 256 buckets, d <= 128 columns");
    return sh;
}

// A gradient or upstream tensor that must agree with the forward's V.
void validate_like_v(const char* entry, const char* name, const at::Tensor& t, const at::Tensor& v) {
    ArgCheck(entry).on_gpu(name, t).matches(name, t, "V", v)
        .require(t.sizes() == v.sizes(), name, "has shape " + dims(t) + ", V " + dims(v))
        .raise();
}

race_options make_options(int64_t tile_tokens, int64_t kernel, bool allow_decode = false) {
    TORCH_CHECK(tile_tokens >= 0 && tile_tokens % RACE_SUB_CHUNK_TOKENS == 0 &&
                    tile_tokens <= (int64_t(1) << 30),
                "tile_tokens must be 0 (automatic) or a positive multiple of ",
                RACE_SUB_CHUNK_TOKENS, ", got ", tile_tokens);
    if (allow_decode) {
        TORCH_CHECK(kernel >= 0 && kernel <= RACE_KERNEL_MFMA_PRECISE,
                    "kernel must be 0 (auto), 1 (valu), 2 (mfma), 3 (mfma_wg), 4 (decode), 5 (single) "
                    "or 6 (mfma_precise)");
    } else {
        TORCH_CHECK(kernel >= 0 && kernel <= RACE_KERNEL_MFMA_PRECISE && kernel != RACE_KERNEL_DECODE,
                    "kernel must be 0 (auto), 1 (valu), 2 (mfma), 3 (mfma_wg), 5 (single) or 6 (mfma_precise)");
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
    ArgCheck("race_fused_fwd_carry")
        .on_gpu("state", init_state)
        .require(init_state.scalar_type() == at::kFloat && init_state.device() == q.device(), "state",
                 "must be float32 on probsQ's device")
        .require(init_state.dim() == 2 && init_state.size(0) == sh.num_streams &&
                     init_state.size(1) == S * sh.head_dim + S,
                 "state", "has shape " + dims(init_state) + ", not [N, S*d + S] = [" +
                              std::to_string(sh.num_streams) + ", " +
                              std::to_string(S * sh.head_dim + S) + "]")
        .raise();
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
    const race_shape sh = validate(q, k, v, "race_noncausal_backward");
    validate_like_v("race_noncausal_backward", "dOut", grad_out, v);
    const int64_t S = int64_t(sh.num_tables) * sh.num_buckets;
    ArgCheck("race_noncausal_backward")
        .on_gpu("state", state)
        .require(state.scalar_type() == at::kFloat && state.device() == q.device() &&
                     state.numel() == sh.num_streams * (S * sh.head_dim + S),
                 "state", "is not the forward's float32 [N, S*d + S] state on probsQ's device")
        .raise();
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
    else  // empty, but with the tile count the backward expects
        records = at::zeros({N, r.tiles, r.rec}, v.options().dtype(at::kFloat));
    return {r.out, records, r.tile};
}

std::tuple<c10::optional<at::Tensor>, c10::optional<at::Tensor>, c10::optional<at::Tensor>>
causal_backward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                const at::Tensor& grad_out, bool need_q, bool need_k, bool need_v,
                int64_t tile_tokens, int64_t kernel, const c10::optional<at::Tensor>& fwd_records) {
    const race_shape sh = validate(q, k, v, "race_causal_backward");
    validate_like_v("race_causal_backward", "dOut", grad_out, v);
    const race_options opts = make_options(tile_tokens, kernel);
    if (fwd_records) {
        const at::Tensor& rec = *fwd_records;
        TORCH_CHECK(tile_tokens > 0, "saved forward records need the forward's tile length");
        // The layout the forward wrote for this shape at this tile length.
        race_options fwd_opts = opts;
        fwd_opts.kernel = RACE_KERNEL_AUTO;
        size_t bytes = 0;
        int64_t tiles = 0, rec_floats = 0;
        check_status(race_fwd_workspace_bytes(&sh, 1, &fwd_opts, &bytes, &tiles, &rec_floats),
                     "race_fwd_workspace_bytes");
        ArgCheck("race_causal_backward")
            .on_gpu("fwd_records", rec)
            .require(rec.device() == q.device() && rec.scalar_type() == at::kFloat &&
                         rec.dim() == 3 && rec.size(0) == q.size(0),
                     "fwd_records", "is not the forward's float32 [N, tiles, rec] records")
            .require(rec.dim() != 3 || rec.size(1) == tiles, "fwd_records",
                     "has " + std::to_string(rec.dim() == 3 ? rec.size(1) : 0) +
                         " tiles; the tile length " + std::to_string(tile_tokens) + " gives " +
                         std::to_string(tiles))
            .require(rec.dim() != 3 || rec.size(2) == rec_floats, "fwd_records",
                     "has records of " + std::to_string(rec.dim() == 3 ? rec.size(2) : 0) +
                         " floats; this (S, d) needs " + std::to_string(rec_floats))
            .raise();
    }
    const c10::DeviceGuard guard(q.device());
    at::Tensor dq, dk, dv;
    if (need_q) dq = at::empty_like(q);
    if (need_k) dk = at::empty_like(k);
    if (need_v) dv = at::empty_like(v);
    const bool from_records = fwd_records && fwd_records->numel() > 0;
    size_t bytes = 0;
    if (from_records)
        check_status(race_causal_bwd_from_records_workspace_bytes(&sh, &opts, &bytes),
                     "race_causal_bwd_from_records_workspace_bytes");
    else
        check_status(race_causal_bwd_workspace_bytes(&sh, &opts, &bytes),
                     "race_causal_bwd_workspace_bytes");
    at::Tensor ws = at::empty({static_cast<int64_t>((bytes + 3) / 4)}, v.options().dtype(at::kFloat));
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    if (from_records)
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
    ArgCheck c("race_hash_probs");
    c.on_gpu("x", x).dtype_is("x", x, true).require(x.dim() >= 1, "x", "has no feature dimension");
    c.raise();
    const int64_t dk = x.size(-1);
    c.on_gpu("planes_T", planes_T)
        .require(planes_T.scalar_type() == at::kFloat && planes_T.device() == x.device(), "planes_T",
                 "must be float32 on x's device")
        .require(planes_T.dim() == 2 && planes_T.size(0) == dk && planes_T.size(1) == L * K,
                 "planes_T", "has shape " + dims(planes_T) + ", not [d_k, L*K]")
        .raise();
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

// dprobs -> dx of the hashing (race_hash_probs_bwd).
at::Tensor hash_probs_backward(const at::Tensor& x, const at::Tensor& planes_T,
                               const at::Tensor& dprobs, int64_t L, int64_t K) {
    ArgCheck c("race_hash_probs_backward");
    c.on_gpu("x", x).dtype_is("x", x, true).require(x.dim() >= 1, "x", "has no feature dimension");
    c.raise();
    const int64_t dk = x.size(-1);
    std::vector<int64_t> pshape(x.sizes().begin(), x.sizes().end() - 1);
    pshape.push_back(L);
    pshape.push_back(int64_t(1) << K);
    c.on_gpu("planes_T", planes_T)
        .require(planes_T.scalar_type() == at::kFloat && planes_T.device() == x.device(), "planes_T",
                 "must be float32 on x's device")
        .require(planes_T.dim() == 2 && planes_T.size(0) == dk && planes_T.size(1) == L * K,
                 "planes_T", "has shape " + dims(planes_T) + ", not [d_k, L*K]")
        .on_gpu("dprobs", dprobs)
        .matches("dprobs", dprobs, "x", x)
        .require(dprobs.sizes() == at::IntArrayRef(pshape), "dprobs",
                 "has shape " + dims(dprobs) + ", not x's leading dimensions + [L, 2^K]")
        .raise();
    const c10::DeviceGuard guard(x.device());
    at::Tensor dx = at::empty_like(x);
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    check_status(race_hash_probs_bwd(x.data_ptr(), planes_T.data_ptr<float>(), dprobs.data_ptr(),
                                     dx.data_ptr(), x.numel() / std::max<int64_t>(dk, 1),
                                     static_cast<int32_t>(dk), static_cast<int32_t>(L),
                                     static_cast<int32_t>(K),
                                     x.scalar_type() == at::kBFloat16 ? RACE_BF16 : RACE_F32, stream),
                 "race_hash_probs_bwd");
    return dx;
}

// The hashed causal forward's arguments: K, Q, V token rows [N, T, d] of one
// dtype, planes [L * Kp, d] float32 (the reference's race_fused_fwd(K, Q, V,
// planes, L), src/race_fused_fwd.cu:150-171).  Returns the shape and Kp.
std::pair<race_shape, int32_t> hashed_validate(const at::Tensor& k, const at::Tensor& q,
                                               const at::Tensor& v, const at::Tensor& planes,
                                               int64_t L) {
    ArgCheck c("race_fused_fwd_hashed");
    c.require(k.dim() == 3, "K", "has shape " + dims(k) + ", not [N, T, d]")
        .on_gpu("K", k).dtype_is("K", k, true)
        .on_gpu("Q", q).matches("Q", q, "K", k)
        .require(q.sizes() == k.sizes(), "Q", "has shape " + dims(q) + ", K " + dims(k))
        .on_gpu("V", v).matches("V", v, "K", k)
        .require(v.sizes() == k.sizes(), "V", "has shape " + dims(v) + ", K " + dims(k))
        .on_gpu("planes", planes)
        .require(planes.scalar_type() == at::kFloat && planes.device() == k.device(), "planes",
                 "must be float32 on K's device")
        .require(L >= 1 && planes.dim() == 2 && k.dim() == 3 && planes.size(1) == k.size(2) &&
                     planes.size(0) % L == 0 && planes.size(0) / L >= 1 && planes.size(0) / L <= 8,
                 "planes", "has shape " + dims(planes) + ", not [L * K, d] for L = " +
                               std::to_string(L) + " and 1 <= K <= 8");
    c.raise();
    const int32_t Kp = static_cast<int32_t>(planes.size(0) / L);
    race_shape sh;
    sh.num_streams = k.size(0);
    sh.seq_len = k.size(1);
    sh.num_tables = static_cast<int32_t>(L);
    sh.num_buckets = 1 << Kp;
    sh.head_dim = static_cast<int32_t>(k.size(2));
    sh.dtype = k.scalar_type() == at::kBFloat16 ? RACE_BF16 : RACE_F32;
    return {sh, Kp};
}

// race_fused_fwd_hashed -> (out, records [N, tiles, rec] or None, state or
// None, tile length).
std::tuple<at::Tensor, c10::optional<at::Tensor>, c10::optional<at::Tensor>, int64_t> hashed_forward(
    const at::Tensor& k, const at::Tensor& q, const at::Tensor& v, const at::Tensor& planes, int64_t L,
    int64_t tile_tokens, bool want_records, bool want_state) {
    const auto [sh, Kp] = hashed_validate(k, q, v, planes, L);
    const race_options opts = make_options(tile_tokens, RACE_KERNEL_AUTO);
    size_t bytes = 0;
    int64_t tiles = 0, rec = 0;
    const race_status st = race_hashed_fwd_workspace_bytes(&sh, Kp, &opts, &bytes, &tiles, &rec);
    TORCH_CHECK(st == RACE_SUCCESS, "race_fused_fwd_hashed: no kernel takes L=", L, ", K=", Kp,
                ", d=", sh.head_dim, " (the hashed kernels need K >= 2, L*K <= 64, L*2^K in ",
                "{64, 128, 256} and d in {64, 128}): ", race_status_string(st));
    const c10::DeviceGuard guard(k.device());
    at::Tensor out = at::empty_like(v);
    const int64_t S = int64_t(sh.num_tables) * sh.num_buckets;
    at::Tensor state;
    if (want_state)
        state = at::empty({sh.num_streams, S * sh.head_dim + S}, v.options().dtype(at::kFloat));
    at::Tensor ws = at::empty({static_cast<int64_t>((bytes + 3) / 4)}, v.options().dtype(at::kFloat));
    int32_t tile = 0;
    race_options wg = opts;
    wg.kernel = RACE_KERNEL_MFMA_WG;
    check_status(race_select_tile_tokens(&sh, 1, &wg, &tile), "race_select_tile_tokens");
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
    check_status(race_hashed_fwd(k.data_ptr(), q.data_ptr(), v.data_ptr(), planes.data_ptr<float>(),
                                 out.data_ptr(), want_state ? state.data_ptr<float>() : nullptr, &sh, Kp,
                                 &opts, ws.data_ptr(), bytes, stream),
                 "race_hashed_fwd");
    c10::optional<at::Tensor> records, st_out;
    if (want_records) {
        const int64_t N = sh.num_streams;
        records = (tiles > 0 && N > 0) ? ws.narrow(0, 0, N * tiles * rec).view({N, tiles, rec})
                                       : at::zeros({N, tiles, rec}, v.options().dtype(at::kFloat));
    }
    if (want_state) st_out = state;
    return {out, records, st_out, tile};
}

// Whether the hashed forward has kernels for (L, K, d).  Host logic only.
bool hashed_supported(int64_t L, int64_t K, int64_t d) {
    if (L < 1 || K < 1 || K > 8 || d < 1) return false;
    race_shape sh{1, 1, static_cast<int32_t>(L), static_cast<int32_t>(1 << K), static_cast<int32_t>(d),
                  RACE_F32};
    race_options o{RACE_SUB_CHUNK_TOKENS, RACE_KERNEL_AUTO};
    size_t bytes = 0;
    return race_hashed_fwd_workspace_bytes(&sh, static_cast<int32_t>(K), &o, &bytes, nullptr, nullptr) ==
           RACE_SUCCESS;
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

// The reference binding's limits for Algorithm 1 (race_causal_fwd.h:45-47),
// applied by the C ABI (race_alg1_shape_supported); this wraps that query
// with a message listing them.
race_alg1_shape alg1_make_shape(int64_t batch_heads, int64_t seq_len, int64_t head_dim,
                                int64_t num_planes, int64_t num_tables) {
    race_alg1_shape sh;
    sh.batch_heads = batch_heads;
    sh.seq_len = seq_len;
    sh.head_dim = static_cast<int32_t>(std::clamp<int64_t>(head_dim, -1, 1 << 20));
    sh.num_planes = static_cast<int32_t>(std::clamp<int64_t>(num_planes, -1, 1 << 20));
    sh.num_tables = static_cast<int32_t>(std::clamp<int64_t>(num_tables, -1, 1 << 20));
    int32_t ok = 0;
    check_status(race_alg1_shape_supported(&sh, &ok), "race_alg1_shape_supported");
    TORCH_CHECK(ok, "causal_v2: no Algorithm-1 kernel for batch*heads=", batch_heads,
                ", tokens=", seq_len, ", head_dim=", head_dim, ", num_planes=", num_planes,
                ", num_tables=", num_tables, " (supported: head_dim 64 or 128, num_planes 1..5, ",
                "num_tables 1..4, batch*heads <= 65535, tokens < 2^31 - ",
                RACE_ALG1_MAX_AUTO_TILE + 1, ")");
    return sh;
}

// q, k, v: bf16 token rows [B, H, T, D] of one shape; W: float32 [L, P, D]
// hash planes; beta: one floating-point value (any device).
race_alg1_shape alg1_validate(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                              const at::Tensor& W, const at::Tensor& beta) {
    ArgCheck c("causal_v2.forward");
    const std::pair<const char*, const at::Tensor*> rows[] = {{"q", &q}, {"k", &k}, {"v", &v}};
    for (const auto& [name, t] : rows)
        c.on_gpu(name, *t).dtype_is(name, *t, false).matches(name, *t, "q", q)
            .require(t->dim() == 4 && t->sizes() == q.sizes(), name,
                     "has shape " + dims(*t) + "; q, k and v are [B, H, T, D] of one shape");
    c.on_gpu("W", W)
        .require(W.scalar_type() == at::kFloat && W.device() == q.device(), "W",
                 "must be float32 on q's device")
        .require(W.dim() == 3 && q.dim() == 4 && W.size(2) == q.size(3), "W",
                 "has shape " + dims(W) + ", not [L, P, D] with q's D")
        .require(beta.numel() == 1 && at::isFloatingType(beta.scalar_type()), "beta",
                 "must be a single floating-point value")
        .raise();
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
    TORCH_CHECK(bytes <= size_t(limit), "causal_v2: ", limit, " bytes of LDS per workgroup on ",
                "this GPU are fewer than the ", bytes, " an Algorithm-1 output-pass workgroup holds ",
                "at (head_dim, num_planes, num_tables) = (", sh.head_dim, ", ", sh.num_planes, ", ",
                sh.num_tables, ")");
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
    m.def("hash_probs_backward", &hash_probs_backward,
          "Gradient of hash_probs w.r.t. the rows: (x, planes_T, dprobs, L, K) -> dx", py::arg("x"),
          py::arg("planes_T"), py::arg("dprobs"), py::arg("L"), py::arg("K"));
    m.def("hashed_forward", &hashed_forward,
          "race_fused_fwd_hashed(K, Q, V, planes, L): the causal op with the hashing inside "
          "-> (out, records or None, state or None, tile length)",
          py::arg("K"), py::arg("Q"), py::arg("V"), py::arg("planes"), py::arg("L"),
          py::arg("tile_tokens") = 0, py::arg("want_records") = false, py::arg("want_state") = false);
    m.def("hashed_supported", &hashed_supported,
          "Whether the hashed causal forward has kernels for (L, K, d)", py::arg("L"), py::arg("K"),
          py::arg("d"));
    m.def("select_tile_tokens", &select_tile_tokens, "Tile length a forward would use",
          py::arg("N"), py::arg("T"), py::arg("L"), py::arg("R"), py::arg("d"),
          py::arg("bf16") = false, py::arg("causal") = true, py::arg("tile_tokens") = 0,
          py::arg("kernel") = 0);
    m.def("shape_supported", &shape_supported, "(supported, has_mfma) for (L, R, d)", py::arg("L"),
          py::arg("R"), py::arg("d"));
    m.def("alg1_forward", &alg1_forward,
          "Algorithm-1 causal attention, hashing inside the kernels -> out [B, H, T, D] bf16",
          py::arg("q"),
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
    m.def("alg1_sub_chunk_tokens", &alg1_sub_chunk_tokens,
          "Tokens per step of the Algorithm-1 kernels (tile lengths are multiples of it)",
          py::arg("head_dim"), py::arg("num_planes"), py::arg("tensor_cores") = false);
    m.def("alg1_select_tile_tokens", &alg1_select_tile_tokens,
          "Automatic Algorithm-1 tile length for this shape on the current GPU",
          py::arg("batch_heads"), py::arg("seq_len"), py::arg("head_dim"), py::arg("num_planes"),
          py::arg("num_tables"), py::arg("tensor_cores") = false);
    m.def("alg1_output_lds_bytes", &alg1_output_lds_bytes,
          "LDS bytes one Algorithm-1 output-pass workgroup allocates",
          py::arg("head_dim"), py::arg("num_planes"), py::arg("num_tables"),
          py::arg("tensor_cores") = false);
    m.def("alg1_fits_on_device", &alg1_fits_on_device,
          "True when an Algorithm-1 output-pass workgroup fits this GPU's LDS", py::arg("head_dim"), py::arg("num_planes"),
          py::arg("num_tables"), py::arg("tensor_cores") = false);
    m.def("abi_version", &race_abi_version, "ABI version of the loaded librace_mi355x");
}
