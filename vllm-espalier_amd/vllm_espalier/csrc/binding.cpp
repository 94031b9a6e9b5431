// espalier_ext: the torch extension module of the plugin, a thin layer over the C ABI in libespalier_hip.so.
//
// The 13 functions, their positional arguments and their checks are those of the reference module
// (vllm_espalier/csrc/experts.cpp:39-248): tensors are checked here (device, dtype, contiguity, sizes) and passed to
// the esp_* entry points as pointers and sizes, on the current stream of the tensor's device. A failing check or call
// raises RuntimeError (c10::Error), as TORCH_CHECK does in the reference.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <vector>

#include "../../../include/espalier.h"

namespace {

void check(const at::Tensor& x, at::ScalarType t, const char* name) {
    TORCH_CHECK(x.is_cuda() && x.scalar_type() == t && x.is_contiguous(), name,
                ": expected a contiguous CUDA tensor of the right dtype");
}

void* cur_stream() { return (void*)c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(); }

int dtype_code(const at::Tensor& t) {
    return t.scalar_type() == at::kFloat ? ESP_F32 : t.scalar_type() == at::kBFloat16 ? ESP_BF16 : ESP_F16;
}

void call(int rc) { TORCH_CHECK(rc == ESP_OK, esp_last_error()); }

template <typename T>
const T* cptr(const at::Tensor& t) { return reinterpret_cast<const T*>(t.data_ptr()); }
template <typename T>
T* mptr(const at::Tensor& t) { return reinterpret_cast<T*>(t.data_ptr()); }

}  // namespace

void grouped(const at::Tensor& X0, const at::Tensor& X1, const at::Tensor& TP0, const at::Tensor& TP1,
             const at::Tensor& B0, const at::Tensor& B1, const at::Tensor& C0, const at::Tensor& C1,
             const at::Tensor& uids, const at::Tensor& ucount, const at::Tensor& members, at::Tensor Z, int64_t mats,
             int64_t K, int64_t N, int64_t P, int64_t SK, int64_t slots, int64_t nt, int64_t warps, int64_t pf,
             int64_t lo, int64_t hi) {
    check(X0, at::kHalf, "X0");
    check(X1, at::kHalf, "X1");
    check(TP0, at::kLong, "TP0");
    check(TP1, at::kLong, "TP1");
    check(B0, at::kInt, "B0");
    check(B1, at::kInt, "B1");
    check(C0, at::kInt, "C0");
    check(C1, at::kInt, "C1");
    check(uids, at::kInt, "uids");
    check(ucount, at::kInt, "ucount");
    check(members, at::kInt, "members");
    check(Z, at::kFloat, "Z");
    TORCH_CHECK(Z.numel() >= mats * SK * P * N, "Z too small");
    TORCH_CHECK(X0.numel() >= P * K && X1.numel() >= P * K, "X too small");
    TORCH_CHECK(members.dim() == 2 && members.size(0) >= uids.numel(), "members: [nexp_max, maxm]");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(X0.device());
    call(esp_grouped(X0.data_ptr(), X1.data_ptr(), cptr<int64_t>(TP0), cptr<int64_t>(TP1), cptr<int32_t>(B0),
                     cptr<int32_t>(B1), cptr<int32_t>(C0), cptr<int32_t>(C1), cptr<int32_t>(uids), uids.numel(),
                     cptr<int32_t>(ucount), cptr<int32_t>(members), members.size(1), mptr<float>(Z), Z.numel(), mats,
                     K, N, P, SK, slots, nt, warps, pf, lo, hi, cur_stream()));
}

// esp_tile_list: the non-empty (expert slot, member tile) pairs of a grouping, for grouped_list
void tile_list(const at::Tensor& ucount, const at::Tensor& members, int64_t nexp_max, int64_t P, at::Tensor tiles) {
    check(ucount, at::kInt, "ucount");
    check(members, at::kInt, "members");
    check(tiles, at::kInt, "tiles");
    TORCH_CHECK(members.dim() == 2 && members.size(0) >= nexp_max, "members: [nexp_max, maxm]");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(members.device());
    call(esp_tile_list(cptr<int32_t>(ucount), cptr<int32_t>(members), nexp_max, members.size(1), P,
                       mptr<int32_t>(tiles), tiles.numel(), cur_stream()));
}

// esp_grouped_list: grouped's programs over tile_list's entries only (the same bits)
void grouped_list(const at::Tensor& X0, const at::Tensor& X1, const at::Tensor& TP0, const at::Tensor& TP1,
                  const at::Tensor& B0, const at::Tensor& B1, const at::Tensor& C0, const at::Tensor& C1,
                  const at::Tensor& uids, const at::Tensor& ucount, const at::Tensor& members,
                  const at::Tensor& tiles, at::Tensor Z, int64_t mats, int64_t K, int64_t N, int64_t P, int64_t SK,
                  int64_t slots, int64_t warps, int64_t lo, int64_t hi) {
    check(X0, at::kHalf, "X0");
    check(X1, at::kHalf, "X1");
    check(TP0, at::kLong, "TP0");
    check(TP1, at::kLong, "TP1");
    check(B0, at::kInt, "B0");
    check(B1, at::kInt, "B1");
    check(C0, at::kInt, "C0");
    check(C1, at::kInt, "C1");
    check(uids, at::kInt, "uids");
    check(ucount, at::kInt, "ucount");
    check(members, at::kInt, "members");
    check(tiles, at::kInt, "tiles");
    check(Z, at::kFloat, "Z");
    TORCH_CHECK(Z.numel() >= mats * SK * P * N, "Z too small");
    TORCH_CHECK(X0.numel() >= P * K && X1.numel() >= P * K, "X too small");
    TORCH_CHECK(members.dim() == 2 && members.size(0) >= uids.numel(), "members: [nexp_max, maxm]");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(X0.device());
    call(esp_grouped_list(X0.data_ptr(), X1.data_ptr(), cptr<int64_t>(TP0), cptr<int64_t>(TP1), cptr<int32_t>(B0),
                          cptr<int32_t>(B1), cptr<int32_t>(C0), cptr<int32_t>(C1), cptr<int32_t>(uids), uids.numel(),
                          cptr<int32_t>(ucount), cptr<int32_t>(members), members.size(1), cptr<int32_t>(tiles),
                          mptr<float>(Z), Z.numel(), mats, K, N, P, SK, slots, warps, lo, hi, cur_stream()));
}

void dequant(const at::Tensor& T, at::Tensor out, int64_t k2, int64_t cb) {
    TORCH_CHECK(T.is_cuda() && T.scalar_type() == at::kShort && T.is_contiguous() && T.dim() == 3,
                "T: int16 [K/16, N/16, 8 * k2]");
    TORCH_CHECK(T.size(2) == 8 * k2, "trellis last dim must be 8 * k2");
    check(out, at::kHalf, "out");
    const int64_t K = T.size(0) * 16, N = T.size(1) * 16;
    TORCH_CHECK(out.numel() == K * N, "out must be [K, N]");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(T.device());
    call(esp_dequant(T.data_ptr(), out.data_ptr(), K, N, k2, cb, cur_stream()));
}

void group(const at::Tensor& pick, at::Tensor uids, at::Tensor ucount, at::Tensor members, int64_t R, int64_t slots,
           int64_t E) {
    check(pick, at::kInt, "pick");
    check(uids, at::kInt, "uids");
    check(ucount, at::kInt, "ucount");
    check(members, at::kInt, "members");
    TORCH_CHECK(pick.numel() >= R * slots, "pick too small");
    TORCH_CHECK(uids.numel() >= std::min<int64_t>(R * slots, E), "uids too small");
    TORCH_CHECK(members.size(0) >= uids.numel() && members.size(1) >= 1, "members too small");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(pick.device());
    call(esp_group(cptr<int32_t>(pick), mptr<int32_t>(uids), uids.numel(), mptr<int32_t>(ucount),
                   mptr<int32_t>(members), members.size(1), R, slots, E, cur_stream()));
}

void rot_in(const at::Tensor& x, int64_t x_stride, const at::Tensor& pick, const at::Tensor& suh0,
            const at::Tensor& suh1, at::Tensor out0, at::Tensor out1, int64_t rows, int64_t K, int64_t slots,
            int64_t E) {
    TORCH_CHECK(x.is_cuda() && (x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf),
                "x: bf16/fp16 CUDA");
    check(pick, at::kInt, "pick");
    check(suh0, at::kHalf, "suh0");
    check(suh1, at::kHalf, "suh1");
    check(out0, at::kHalf, "out0");
    check(out1, at::kHalf, "out1");
    TORCH_CHECK(K % 128 == 0, "K must be a multiple of 128");
    TORCH_CHECK(pick.numel() >= rows * slots, "pick too small");
    TORCH_CHECK(out0.numel() >= rows * slots * K && out1.numel() >= rows * slots * K, "out too small");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    call(esp_rot_in(x.data_ptr(), dtype_code(x), x_stride, cptr<int32_t>(pick), suh0.data_ptr(), suh1.data_ptr(),
                    out0.data_ptr(), out1.data_ptr(), rows, K, slots, E, cur_stream()));
}

void gateup_epilogue(const at::Tensor& Z, const at::Tensor& pick, const at::Tensor& svh_g, const at::Tensor& svh_u,
                     const at::Tensor& suh_d, at::Tensor xd, int64_t rows, int64_t P, int64_t N, int64_t SK,
                     int64_t slots, int64_t E, double limit, int64_t act_mode) {
    check(Z, at::kFloat, "Z");
    check(pick, at::kInt, "pick");
    check(svh_g, at::kHalf, "svh_g");
    check(svh_u, at::kHalf, "svh_u");
    check(suh_d, at::kHalf, "suh_d");
    check(xd, at::kHalf, "xd");
    TORCH_CHECK(N % 128 == 0, "N must be a multiple of 128");
    TORCH_CHECK(Z.numel() >= 2 * SK * P * N && xd.numel() >= rows * slots * N, "Z / xd too small");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(Z.device());
    call(esp_gateup_epilogue(cptr<float>(Z), cptr<int32_t>(pick), svh_g.data_ptr(), svh_u.data_ptr(),
                             suh_d.data_ptr(), xd.data_ptr(), rows, P, N, SK, slots, E, limit, act_mode,
                             cur_stream()));
}

void down_epilogue(const at::Tensor& Z, const at::Tensor& pick, const at::Tensor& svh_d, at::Tensor y, int64_t rows,
                   int64_t P, int64_t D, int64_t SK, int64_t slots, int64_t E) {
    check(Z, at::kFloat, "Z");
    check(pick, at::kInt, "pick");
    check(svh_d, at::kHalf, "svh_d");
    check(y, at::kFloat, "y");
    TORCH_CHECK(D % 128 == 0, "D must be a multiple of 128");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(Z.device());
    call(esp_down_epilogue(cptr<float>(Z), cptr<int32_t>(pick), svh_d.data_ptr(), mptr<float>(y), rows, P, D, SK,
                           slots, E, cur_stream()));
}

void combine(const at::Tensor& y, const at::Tensor& wts, at::Tensor out, int64_t rows, int64_t D, int64_t slots) {
    check(y, at::kFloat, "y");
    check(wts, at::kFloat, "wts");
    check(out, at::kFloat, "out");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(y.device());
    call(esp_combine(cptr<float>(y), cptr<float>(wts), mptr<float>(out), rows, D, slots, cur_stream()));
}

void down_combine(const at::Tensor& Z, const at::Tensor& pick, const at::Tensor& svh_d, at::Tensor y,
                  const at::Tensor& wts, at::Tensor out, int64_t rows, int64_t P, int64_t D, int64_t SK, int64_t slots,
                  int64_t E) {
    check(Z, at::kFloat, "Z");
    check(pick, at::kInt, "pick");
    check(svh_d, at::kHalf, "svh_d");
    check(y, at::kFloat, "y");
    check(wts, at::kFloat, "wts");
    check(out, at::kFloat, "out");
    TORCH_CHECK(D % 128 == 0, "D must be a multiple of 128");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(Z.device());
    call(esp_down_combine(cptr<float>(Z), cptr<int32_t>(pick), svh_d.data_ptr(), mptr<float>(y), cptr<float>(wts),
                          mptr<float>(out), rows, P, D, SK, slots, E, cur_stream()));
}

void group_shared(const at::Tensor& pick_in, const at::Tensor& wts_in, const at::Tensor& x, int64_t x_stride,
                  const c10::optional<at::Tensor>& gate_w, int64_t shared_id, at::Tensor pick_out, at::Tensor wts_out,
                  at::Tensor uids, at::Tensor ucount, at::Tensor members, int64_t R, int64_t slots_in, int64_t E) {
    check(pick_in, at::kInt, "pick_in");
    check(wts_in, at::kFloat, "wts_in");
    check(pick_out, at::kInt, "pick_out");
    check(wts_out, at::kFloat, "wts_out");
    check(uids, at::kInt, "uids");
    check(ucount, at::kInt, "ucount");
    check(members, at::kInt, "members");
    TORCH_CHECK(x.is_cuda() && (x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf),
                "x: bf16/fp16 CUDA");
    if (gate_w.has_value())
        TORCH_CHECK(gate_w->scalar_type() == x.scalar_type() && gate_w->is_contiguous() && gate_w->numel() == x.size(1),
                    "gate_w: x's dtype, [H]");
    TORCH_CHECK(shared_id < 0 || gate_w.has_value(), "a shared slot needs its gate weight");
    TORCH_CHECK(members.dim() == 2, "members: [nexp_max, maxm]");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    call(esp_group_shared(cptr<int32_t>(pick_in), cptr<float>(wts_in), x.data_ptr(), dtype_code(x), x_stride,
                          x.size(1), gate_w.has_value() ? gate_w->data_ptr() : nullptr, shared_id,
                          mptr<int32_t>(pick_out), mptr<float>(wts_out), mptr<int32_t>(uids), uids.numel(),
                          mptr<int32_t>(ucount), mptr<int32_t>(members), members.size(1), R, slots_in, E,
                          cur_stream()));
}

void down_combine2(const at::Tensor& Z, const at::Tensor& pick, const at::Tensor& svh_d,
                   const c10::optional<at::Tensor>& y, const at::Tensor& wts, at::Tensor out,
                   const c10::optional<at::Tensor>& out_shared, int64_t rows, int64_t P, int64_t D, int64_t SK,
                   int64_t slots, int64_t E, int64_t n_routed) {
    check(Z, at::kFloat, "Z");
    check(pick, at::kInt, "pick");
    check(svh_d, at::kHalf, "svh_d");
    if (y.has_value()) check(*y, at::kFloat, "y");   // None: no per-slot outputs stored (esp_down_combine2)
    check(wts, at::kFloat, "wts");
    TORCH_CHECK(out.is_cuda() && out.is_contiguous(), "out: contiguous CUDA");
    TORCH_CHECK(out.scalar_type() == at::kBFloat16 || out.scalar_type() == at::kHalf ||
                    out.scalar_type() == at::kFloat,
                "out: bf16, fp16 or fp32");
    if (out_shared.has_value())
        TORCH_CHECK(out_shared->scalar_type() == out.scalar_type() && out_shared->is_contiguous(),
                    "out_shared: out's dtype");
    TORCH_CHECK(D % 128 == 0, "D must be a multiple of 128");
    TORCH_CHECK(n_routed <= slots, "n_routed <= slots");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(Z.device());
    call(esp_down_combine2(cptr<float>(Z), cptr<int32_t>(pick), svh_d.data_ptr(),
                           y.has_value() ? mptr<float>(*y) : nullptr, cptr<float>(wts),
                           out.data_ptr(), dtype_code(out), out_shared.has_value() ? out_shared->data_ptr() : nullptr,
                           rows, P, D, SK, slots, E, n_routed, cur_stream()));
}

// dense's checks and call; own: Z is the caller's all-ones partials buffer (esp_dense_own)
static void dense_call(const at::Tensor& x, const std::vector<at::Tensor>& T, const std::vector<at::Tensor>& suh,
                       const std::vector<at::Tensor>& svh, const std::vector<int64_t>& col0, at::Tensor y,
                       at::Tensor xh, at::Tensor Z, at::Tensor counters, int64_t k2, int64_t cb, int64_t SK, int64_t W,
                       int64_t PF, int64_t rot_smem, bool own) {
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.stride(1) == 1, "x: CUDA [M, K], unit column stride");
    TORCH_CHECK(y.is_cuda() && y.dim() == 2 && y.stride(1) == 1, "y: CUDA [M, N], unit column stride");
    TORCH_CHECK(T.size() == suh.size() && T.size() == svh.size() && T.size() == col0.size(), "one entry a matrix");
    TORCH_CHECK(T.size() >= 1 && T.size() <= 4, "1 to 4 matrices a launch");
    const int64_t M = x.size(0), K = x.size(1);
    std::vector<const void*> tp, sp, vp;
    std::vector<int64_t> ncols;
    for (size_t s = 0; s < T.size(); ++s) {
        TORCH_CHECK(T[s].is_cuda() && T[s].scalar_type() == at::kShort && T[s].is_contiguous() && T[s].dim() == 3,
                    "trellis: contiguous int16 [K/16, N/16, 16K]");
        check(suh[s], at::kHalf, "suh");
        check(svh[s], at::kHalf, "svh");
        TORCH_CHECK(col0[s] + svh[s].numel() <= y.size(1), "matrix columns past y");
        TORCH_CHECK(T[s].size(0) * 16 == K && T[s].size(1) * 16 == svh[s].numel() && T[s].size(2) == 8 * k2,
                    "matrix shape");
        TORCH_CHECK(suh[s].numel() == K, "suh must have K elements");
        tp.push_back(T[s].data_ptr());
        sp.push_back(suh[s].data_ptr());
        vp.push_back(svh[s].data_ptr());
        ncols.push_back(svh[s].numel());
    }
    check(Z, at::kFloat, "Z");
    check(counters, at::kInt, "counters");
    TORCH_CHECK(xh.scalar_type() == at::kHalf, "xh: fp16 scratch");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    auto fn = own ? esp_dense_own : esp_dense;
    call(fn(x.data_ptr(), dtype_code(x), x.stride(0), M, K, (int64_t)T.size(), tp.data(), sp.data(), vp.data(),
            ncols.data(), col0.data(), y.data_ptr(), dtype_code(y), y.stride(0), y.size(1), xh.data_ptr(), xh.numel(),
            mptr<float>(Z), Z.numel(), mptr<int32_t>(counters), counters.numel(), k2, cb, SK, W, PF, rot_smem,
            cur_stream()));
}

void dense(const at::Tensor& x, const std::vector<at::Tensor>& T, const std::vector<at::Tensor>& suh,
           const std::vector<at::Tensor>& svh, const std::vector<int64_t>& col0, at::Tensor y, at::Tensor xh,
           at::Tensor Z, at::Tensor counters, int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t PF,
           int64_t rot_smem) {
    dense_call(x, T, suh, svh, col0, y, xh, Z, counters, k2, cb, SK, W, PF, rot_smem, false);
}

// dense over the caller's all-ones partials buffer (esp_dense_own; no reference counterpart)
void dense_own(const at::Tensor& x, const std::vector<at::Tensor>& T, const std::vector<at::Tensor>& suh,
               const std::vector<at::Tensor>& svh, const std::vector<int64_t>& col0, at::Tensor y, at::Tensor xh,
               at::Tensor Z, at::Tensor counters, int64_t k2, int64_t cb, int64_t SK, int64_t W, int64_t PF,
               int64_t rot_smem) {
    dense_call(x, T, suh, svh, col0, y, xh, Z, counters, k2, cb, SK, W, PF, rot_smem, true);
}

// dense over a whole prompt (no reference counterpart): x [T, K], any T
void dense_tile(const at::Tensor& x, const std::vector<at::Tensor>& T, const std::vector<at::Tensor>& suh,
                const std::vector<at::Tensor>& svh, const std::vector<int64_t>& col0, at::Tensor y, at::Tensor xh,
                at::Tensor Z, at::Tensor counters, int64_t k2, int64_t cb, int64_t SK) {
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.stride(1) == 1, "x: CUDA [T, K], unit column stride");
    TORCH_CHECK(y.is_cuda() && y.dim() == 2 && y.stride(1) == 1 && y.size(0) == x.size(0),
                "y: CUDA [T, N], unit column stride");
    TORCH_CHECK(T.size() == suh.size() && T.size() == svh.size() && T.size() == col0.size(), "one entry a matrix");
    TORCH_CHECK(T.size() >= 1 && T.size() <= 4, "1 to 4 matrices a launch");
    const int64_t M = x.size(0), K = x.size(1);
    std::vector<const void*> tp, sp, vp;
    std::vector<int64_t> ncols;
    for (size_t s = 0; s < T.size(); ++s) {
        TORCH_CHECK(T[s].is_cuda() && T[s].scalar_type() == at::kShort && T[s].is_contiguous() && T[s].dim() == 3,
                    "trellis: contiguous int16 [K/16, N/16, 16K]");
        check(suh[s], at::kHalf, "suh");
        check(svh[s], at::kHalf, "svh");
        TORCH_CHECK(T[s].size(0) * 16 == K && T[s].size(1) * 16 == svh[s].numel() && T[s].size(2) == 8 * k2,
                    "matrix shape");
        TORCH_CHECK(suh[s].numel() == K, "suh must have K elements");
        tp.push_back(T[s].data_ptr());
        sp.push_back(suh[s].data_ptr());
        vp.push_back(svh[s].data_ptr());
        ncols.push_back(svh[s].numel());
    }
    check(Z, at::kFloat, "Z");
    check(counters, at::kInt, "counters");
    check(xh, at::kHalf, "xh");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    call(esp_dense_tile(x.data_ptr(), dtype_code(x), x.stride(0), M, K, (int64_t)T.size(), tp.data(), sp.data(),
                        vp.data(), ncols.data(), col0.data(), y.data_ptr(), dtype_code(y), y.stride(0), y.size(1),
                        xh.data_ptr(), xh.numel(), mptr<float>(Z), Z.numel(), mptr<int32_t>(counters),
                        counters.numel(), k2, cb, SK, cur_stream()));
}

// route_group's checks and call; own: over the caller's all-ones logits buffer (esp_route_group_own)
static void route_group_impl(const at::Tensor& x, const at::Tensor& gate, const c10::optional<at::Tensor>& sgate,
                             int64_t k, int64_t shared_id, at::Tensor logits, at::Tensor counter, at::Tensor pick_out,
                             at::Tensor wts_out, at::Tensor uids, at::Tensor ucount, at::Tensor members, bool own) {
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.stride(1) == 1 && gate.is_contiguous(), "x / gate layout");
    TORCH_CHECK(gate.scalar_type() == x.scalar_type(), "gate and x must share a dtype");
    TORCH_CHECK(x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf, "x: bf16/fp16");
    check(logits, at::kFloat, "logits");
    check(counter, at::kInt, "counter");
    check(pick_out, at::kInt, "pick_out");
    check(wts_out, at::kFloat, "wts_out");
    check(uids, at::kInt, "uids");
    check(ucount, at::kInt, "ucount");
    check(members, at::kInt, "members");
    TORCH_CHECK(members.dim() == 2, "members: [nexp_max, maxm]");
    TORCH_CHECK(gate.dim() == 2 && gate.size(1) == x.size(1), "gate: [E, H]");
    if (sgate.has_value())
        TORCH_CHECK(sgate->scalar_type() == x.scalar_type() && sgate->is_contiguous() && sgate->numel() == x.size(1),
                    "sgate: x's dtype, [H]");
    const int64_t R = x.size(0), H = x.size(1), E = gate.size(0);
    const int64_t slots = k + (shared_id >= 0);
    TORCH_CHECK(pick_out.numel() >= R * slots && wts_out.numel() >= R * slots, "pick / wts too small");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    auto fn = own ? esp_route_group_own : esp_route_group;
    call(fn(x.data_ptr(), dtype_code(x), x.stride(0), R, H, gate.data_ptr(), E,
            sgate.has_value() ? sgate->data_ptr() : nullptr, k, shared_id, mptr<float>(logits), logits.numel(),
            mptr<int32_t>(counter), mptr<int32_t>(pick_out), mptr<float>(wts_out), mptr<int32_t>(uids), uids.numel(),
            mptr<int32_t>(ucount), mptr<int32_t>(members), members.size(1), cur_stream()));
}

void route_group(const at::Tensor& x, const at::Tensor& gate, const c10::optional<at::Tensor>& sgate, int64_t k,
                 int64_t shared_id, at::Tensor logits, at::Tensor counter, at::Tensor pick_out, at::Tensor wts_out,
                 at::Tensor uids, at::Tensor ucount, at::Tensor members) {
    route_group_impl(x, gate, sgate, k, shared_id, logits, counter, pick_out, wts_out, uids, ucount, members, false);
}

// route_group over its own all-ones logits buffer (esp_route_group_own; no reference counterpart)
void route_group_own(const at::Tensor& x, const at::Tensor& gate, const c10::optional<at::Tensor>& sgate, int64_t k,
                     int64_t shared_id, at::Tensor logits, at::Tensor counter, at::Tensor pick_out,
                     at::Tensor wts_out, at::Tensor uids, at::Tensor ucount, at::Tensor members) {
    route_group_impl(x, gate, sgate, k, shared_id, logits, counter, pick_out, wts_out, uids, ucount, members, true);
}

// route_group's routing over any number of rows, without the grouping (no reference counterpart)
void route_rows(const at::Tensor& x, const at::Tensor& gate, const c10::optional<at::Tensor>& sgate, int64_t k,
                int64_t shared_id, at::Tensor logits, at::Tensor pick_out, at::Tensor wts_out) {
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.stride(1) == 1 && gate.is_contiguous(), "x / gate layout");
    TORCH_CHECK(gate.scalar_type() == x.scalar_type(), "gate and x must share a dtype");
    check(logits, at::kFloat, "logits");
    check(pick_out, at::kInt, "pick_out");
    check(wts_out, at::kFloat, "wts_out");
    TORCH_CHECK(gate.dim() == 2 && gate.size(1) == x.size(1), "gate: [E, H]");
    if (sgate.has_value())
        TORCH_CHECK(sgate->scalar_type() == x.scalar_type() && sgate->is_contiguous() && sgate->numel() == x.size(1),
                    "sgate: x's dtype, [H]");
    const int64_t R = x.size(0), H = x.size(1), E = gate.size(0);
    const int64_t slots = k + (shared_id >= 0);
    TORCH_CHECK(pick_out.numel() >= R * slots && wts_out.numel() >= R * slots, "pick / wts too small");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    call(esp_route_rows(x.data_ptr(), dtype_code(x), x.stride(0), R, H, gate.data_ptr(), E,
                        sgate.has_value() ? sgate->data_ptr() : nullptr, k, shared_id, mptr<float>(logits),
                        logits.numel(), mptr<int32_t>(pick_out), mptr<float>(wts_out), cur_stream()));
}

// dense with its input rows normalised in the launch (no reference counterpart): h, d1, d2 [M, K] contiguous rows
void dense_rmsnorm(const at::Tensor& h, const c10::optional<at::Tensor>& d1, const c10::optional<at::Tensor>& d2,
                   const at::Tensor& norm_w, double eps, at::Tensor h_out, const std::vector<at::Tensor>& T,
                   const std::vector<at::Tensor>& suh, const std::vector<at::Tensor>& svh,
                   const std::vector<int64_t>& col0, at::Tensor y, at::Tensor Z, at::Tensor counters, int64_t k2,
                   int64_t cb, int64_t SK, int64_t W, int64_t rot_smem) {
    TORCH_CHECK(h.is_cuda() && h.dim() == 2 && h.is_contiguous(), "h: CUDA [M, K] contiguous");
    const auto t = h.scalar_type();
    TORCH_CHECK(t == at::kBFloat16 || t == at::kHalf, "h: bf16/fp16");
    for (const auto* d : {&d1, &d2})
        if (d->has_value()) TORCH_CHECK((*d)->is_contiguous() && (*d)->scalar_type() == t && (*d)->sizes() == h.sizes(),
                                        "deltas: h's dtype and shape, contiguous");
    check(norm_w, t, "norm_w");
    check(h_out, t, "h_out");
    TORCH_CHECK(norm_w.numel() == h.size(1) && h_out.sizes() == h.sizes(), "norm_w: [K]; h_out: h's shape");
    TORCH_CHECK(y.is_cuda() && y.dim() == 2 && y.stride(1) == 1, "y: CUDA [M, N], unit column stride");
    TORCH_CHECK(T.size() == suh.size() && T.size() == svh.size() && T.size() == col0.size(), "one entry a matrix");
    TORCH_CHECK(T.size() >= 1 && T.size() <= 4, "1 to 4 matrices a launch");
    const int64_t M = h.size(0), K = h.size(1);
    std::vector<const void*> tp, sp, vp;
    std::vector<int64_t> ncols;
    for (size_t s = 0; s < T.size(); ++s) {
        TORCH_CHECK(T[s].is_cuda() && T[s].scalar_type() == at::kShort && T[s].is_contiguous() && T[s].dim() == 3,
                    "trellis: contiguous int16 [K/16, N/16, 16K]");
        check(suh[s], at::kHalf, "suh");
        check(svh[s], at::kHalf, "svh");
        TORCH_CHECK(col0[s] + svh[s].numel() <= y.size(1), "matrix columns past y");
        TORCH_CHECK(T[s].size(0) * 16 == K && T[s].size(1) * 16 == svh[s].numel() && T[s].size(2) == 8 * k2,
                    "matrix shape");
        TORCH_CHECK(suh[s].numel() == K, "suh must have K elements");
        tp.push_back(T[s].data_ptr());
        sp.push_back(suh[s].data_ptr());
        vp.push_back(svh[s].data_ptr());
        ncols.push_back(svh[s].numel());
    }
    check(Z, at::kFloat, "Z");
    check(counters, at::kInt, "counters");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(h.device());
    call(esp_dense_rmsnorm(h.data_ptr(), d1.has_value() ? d1->data_ptr() : nullptr,
                           d2.has_value() ? d2->data_ptr() : nullptr, norm_w.data_ptr(), eps, h_out.data_ptr(),
                           dtype_code(h), h.stride(0), M, K, (int64_t)T.size(), tp.data(), sp.data(), vp.data(),
                           ncols.data(), col0.data(), y.data_ptr(), dtype_code(y), y.stride(0), y.size(1),
                           mptr<float>(Z), Z.numel(), mptr<int32_t>(counters), counters.numel(), k2, cb, SK, W,
                           rot_smem, cur_stream()));
}

// route_group with its input normalised in the launch (no reference counterpart): x = RMSNorm(h + d1) * norm_w
void route_group_rmsnorm(const at::Tensor& h, const c10::optional<at::Tensor>& d1, const at::Tensor& norm_w,
                         double eps, at::Tensor h_out, at::Tensor a_out, const at::Tensor& gate,
                         const c10::optional<at::Tensor>& sgate, int64_t k, int64_t shared_id, at::Tensor logits,
                         at::Tensor counter, at::Tensor pick_out, at::Tensor wts_out, at::Tensor uids,
                         at::Tensor ucount, at::Tensor members) {
    TORCH_CHECK(h.is_cuda() && h.dim() == 2 && h.is_contiguous() && gate.is_contiguous(), "h / gate layout");
    const auto t = h.scalar_type();
    TORCH_CHECK(t == at::kBFloat16 || t == at::kHalf, "h: bf16/fp16");
    TORCH_CHECK(gate.scalar_type() == t, "gate and h must share a dtype");
    if (d1.has_value())
        TORCH_CHECK(d1->is_contiguous() && d1->scalar_type() == t && d1->sizes() == h.sizes(),
                    "d1: h's dtype and shape");
    check(norm_w, t, "norm_w");
    check(h_out, t, "h_out");
    check(a_out, t, "a_out");
    TORCH_CHECK(norm_w.numel() == h.size(1) && h_out.sizes() == h.sizes() && a_out.sizes() == h.sizes(),
                "norm_w: [H]; h_out / a_out: h's shape");
    check(logits, at::kFloat, "logits");
    check(counter, at::kInt, "counter");
    check(pick_out, at::kInt, "pick_out");
    check(wts_out, at::kFloat, "wts_out");
    check(uids, at::kInt, "uids");
    check(ucount, at::kInt, "ucount");
    check(members, at::kInt, "members");
    TORCH_CHECK(members.dim() == 2, "members: [nexp_max, maxm]");
    TORCH_CHECK(gate.dim() == 2 && gate.size(1) == h.size(1), "gate: [E, H]");
    if (sgate.has_value())
        TORCH_CHECK(sgate->scalar_type() == t && sgate->is_contiguous() && sgate->numel() == h.size(1),
                    "sgate: h's dtype, [H]");
    const int64_t R = h.size(0), H = h.size(1), E = gate.size(0);
    const int64_t slots = k + (shared_id >= 0);
    TORCH_CHECK(pick_out.numel() >= R * slots && wts_out.numel() >= R * slots, "pick / wts too small");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(h.device());
    call(esp_route_group_rmsnorm(h.data_ptr(), d1.has_value() ? d1->data_ptr() : nullptr, norm_w.data_ptr(), eps,
                                 h_out.data_ptr(), a_out.data_ptr(), dtype_code(h), h.stride(0), R, H, gate.data_ptr(),
                                 E, sgate.has_value() ? sgate->data_ptr() : nullptr, k, shared_id, mptr<float>(logits),
                                 logits.numel(), mptr<int32_t>(counter), mptr<int32_t>(pick_out),
                                 mptr<float>(wts_out), mptr<int32_t>(uids), uids.numel(), mptr<int32_t>(ucount),
                                 mptr<int32_t>(members), members.size(1), cur_stream()));
}

void had(const at::Tensor& x, const c10::optional<at::Tensor>& pre, const c10::optional<at::Tensor>& post,
         at::Tensor y) {
    check(x, at::kHalf, "x");
    check(y, at::kHalf, "y");
    TORCH_CHECK(x.dim() == 2 && y.numel() == x.numel(), "had: x [M, K], y the same size");
    const int64_t M = x.size(0), K = x.size(1);
    if (pre.has_value()) check(*pre, at::kHalf, "pre");
    if (post.has_value()) check(*post, at::kHalf, "post");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    call(esp_had(x.data_ptr(), pre.has_value() ? pre->data_ptr() : nullptr,
                 post.has_value() ? post->data_ptr() : nullptr, y.data_ptr(), M, K, cur_stream()));
}

// fused gate/up launch (no reference counterpart: rot_in + grouped + gateup_epilogue in one launch)
void moe_gateup(const at::Tensor& x, int64_t x_stride, const at::Tensor& suh_g, const at::Tensor& suh_u,
                const at::Tensor& TP0, const at::Tensor& TP1, const at::Tensor& B0, const at::Tensor& B1,
                const at::Tensor& C0, const at::Tensor& C1, const at::Tensor& uids, const at::Tensor& ucount,
                const at::Tensor& members, at::Tensor Z, at::Tensor counters, const at::Tensor& svh_g,
                const at::Tensor& svh_u, const at::Tensor& suh_d, at::Tensor xd, int64_t K, int64_t N, int64_t P,
                int64_t SK, int64_t slots, int64_t warps, int64_t lo, int64_t hi, double limit, int64_t act_mode) {
    TORCH_CHECK(x.is_cuda() && (x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf) && x.stride(-1) == 1,
                "x: bf16/fp16 rows with unit column stride");
    using TL = std::initializer_list<const at::Tensor*>;
    for (const at::Tensor* t : TL{&suh_g, &suh_u, &svh_g, &svh_u, &suh_d, &xd}) check(*t, at::kHalf, "fp16 table");
    check(TP0, at::kLong, "TP0");
    check(TP1, at::kLong, "TP1");
    for (const at::Tensor* t : TL{&B0, &B1, &C0, &C1, &uids, &ucount, &members, &counters})
        check(*t, at::kInt, "int table");
    check(Z, at::kFloat, "Z");
    TORCH_CHECK(members.dim() == 2 && members.size(0) >= uids.numel(), "members: [nexp_max, maxm]");
    TORCH_CHECK(xd.numel() >= P * N, "xd too small");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    call(esp_moe_gateup(x.data_ptr(), dtype_code(x), x_stride, suh_g.data_ptr(), suh_u.data_ptr(), cptr<int64_t>(TP0),
                        cptr<int64_t>(TP1), cptr<int32_t>(B0), cptr<int32_t>(B1), cptr<int32_t>(C0), cptr<int32_t>(C1),
                        cptr<int32_t>(uids), uids.numel(), cptr<int32_t>(ucount), cptr<int32_t>(members),
                        members.size(1), mptr<float>(Z), Z.numel(), mptr<int32_t>(counters), counters.numel(),
                        svh_g.data_ptr(), svh_u.data_ptr(), suh_d.data_ptr(), xd.data_ptr(), K, N, P, SK, slots, warps,
                        lo, hi, limit, act_mode, cur_stream()));
}

// the chained decode MoE layer (no reference counterpart; esp_moe_chain)
void moe_chain(const at::Tensor& x, int64_t x_stride, const at::Tensor& suh_g, const at::Tensor& suh_u,
               const at::Tensor& TP0, const at::Tensor& TP1, const at::Tensor& TP2, const at::Tensor& B0,
               const at::Tensor& B1, const at::Tensor& B2, const at::Tensor& C0, const at::Tensor& C1,
               const at::Tensor& C2, const at::Tensor& uids, const at::Tensor& ucount, const at::Tensor& members,
               const at::Tensor& pick, const at::Tensor& wts, const at::Tensor& svh_g, const at::Tensor& svh_u,
               const at::Tensor& suh_d, const at::Tensor& svh_d, at::Tensor xd, at::Tensor Z, at::Tensor Zd,
               at::Tensor y, at::Tensor out, std::optional<at::Tensor> out_shared, at::Tensor counters,
               at::Tensor flags, int64_t D, int64_t I, int64_t SK, int64_t slots, int64_t E, int64_t n_routed,
               int64_t lo, int64_t hi, int64_t lo_d, int64_t hi_d, double limit, int64_t act_mode) {
    TORCH_CHECK(x.is_cuda() && (x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf) && x.stride(-1) == 1,
                "x: bf16/fp16 rows with unit column stride");
    using TL = std::initializer_list<const at::Tensor*>;
    for (const at::Tensor* t : TL{&suh_g, &suh_u, &svh_g, &svh_u, &suh_d, &svh_d, &xd}) check(*t, at::kHalf, "fp16 table");
    for (const at::Tensor* t : TL{&TP0, &TP1, &TP2}) check(*t, at::kLong, "pointer table");
    for (const at::Tensor* t : TL{&B0, &B1, &B2, &C0, &C1, &C2, &uids, &ucount, &members, &pick, &counters, &flags})
        check(*t, at::kInt, "int table");
    for (const at::Tensor* t : TL{&wts, &Z, &Zd, &y}) check(*t, at::kFloat, "fp32 buffer");
    TORCH_CHECK(members.dim() == 2 && members.size(0) >= uids.numel(), "members: [nexp_max, rows]");
    const int64_t rows = members.size(1), P = rows * slots;
    TORCH_CHECK(pick.numel() >= P && wts.numel() >= P && xd.numel() >= P * I && y.numel() >= P * D,
                "pick / wts / xd / y too small");
    TORCH_CHECK(out.is_cuda() && out.is_contiguous() && out.numel() >= rows * D, "out: [rows, D] contiguous");
    if (out_shared.has_value())
        TORCH_CHECK(out_shared->is_cuda() && out_shared->is_contiguous() && out_shared->scalar_type() == out.scalar_type() &&
                        out_shared->numel() >= rows * D,
                    "out_shared: out's dtype, [rows, D] contiguous");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    call(esp_moe_chain(x.data_ptr(), dtype_code(x), x_stride, suh_g.data_ptr(), suh_u.data_ptr(), cptr<int64_t>(TP0),
                       cptr<int64_t>(TP1), cptr<int64_t>(TP2), cptr<int32_t>(B0), cptr<int32_t>(B1), cptr<int32_t>(B2),
                       cptr<int32_t>(C0), cptr<int32_t>(C1), cptr<int32_t>(C2), cptr<int32_t>(uids), uids.numel(),
                       cptr<int32_t>(ucount), cptr<int32_t>(members), rows, cptr<int32_t>(pick), cptr<float>(wts),
                       svh_g.data_ptr(), svh_u.data_ptr(), suh_d.data_ptr(), svh_d.data_ptr(), xd.data_ptr(),
                       mptr<float>(Z), Z.numel(), mptr<float>(Zd), Zd.numel(), mptr<float>(y), out.data_ptr(),
                       dtype_code(out), out_shared.has_value() ? out_shared->data_ptr() : nullptr,
                       mptr<int32_t>(counters), counters.numel(), mptr<int32_t>(flags), flags.numel(), D, I, SK, slots,
                       E, n_routed, lo, hi, lo_d, hi_d, limit, act_mode, cur_stream()));
}

// decode-step glue (no reference counterpart; csrc/step.hip)
void embed(const at::Tensor& ids, const at::Tensor& table, at::Tensor h) {
    check(ids, at::kInt, "ids");
    TORCH_CHECK(table.is_cuda() && table.is_contiguous() && table.dim() == 2, "table: [vocab, D] contiguous");
    TORCH_CHECK(h.is_cuda() && h.is_contiguous() && h.scalar_type() == table.scalar_type() && h.dim() == 2 &&
                    h.size(1) == table.size(1) && h.size(0) == ids.numel(),
                "h: [T, D] contiguous, table's dtype, T = ids.numel()");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(h.device());
    call(esp_embed(cptr<int32_t>(ids), table.data_ptr(), table.size(0), h.data_ptr(), h.size(0), h.size(1),
                   cur_stream()));
}

void add_rmsnorm(at::Tensor h, const c10::optional<at::Tensor>& d1, const c10::optional<at::Tensor>& d2,
                 const at::Tensor& w, at::Tensor out, double eps) {
    TORCH_CHECK(h.is_cuda() && h.is_contiguous() && h.dim() == 2, "h: [T, D] contiguous");
    const auto t = h.scalar_type();
    TORCH_CHECK(t == at::kBFloat16 || t == at::kHalf, "h: bf16 or fp16");
    for (const auto* d : {&d1, &d2}) {
        if (!d->has_value()) continue;
        check(**d, t, "delta");
        TORCH_CHECK((*d)->sizes() == h.sizes(), "deltas: h's shape");
    }
    check(w, t, "w");
    check(out, t, "out");
    TORCH_CHECK(w.numel() == h.size(1) && out.sizes() == h.sizes(), "w: [D]; out: h's shape");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(h.device());
    call(esp_add_rmsnorm(h.data_ptr(), d1.has_value() ? d1->data_ptr() : nullptr,
                         d2.has_value() ? d2->data_ptr() : nullptr, w.data_ptr(), out.data_ptr(), h.size(0),
                         h.size(1), eps, dtype_code(h), cur_stream()));
}

void argmax(const at::Tensor& logits, at::Tensor ids, std::optional<at::Tensor> part,
            std::optional<at::Tensor> counters) {
    TORCH_CHECK(logits.is_cuda() && logits.dim() == 2 && logits.stride(1) == 1, "logits: [T, N], unit column stride");
    TORCH_CHECK(logits.scalar_type() == at::kBFloat16 || logits.scalar_type() == at::kHalf, "logits: bf16 or fp16");
    check(ids, at::kInt, "ids");
    TORCH_CHECK(ids.numel() == logits.size(0), "ids: [T]");
    TORCH_CHECK(part.has_value() == counters.has_value(), "argmax: part and counters go together");
    if (part.has_value()) {
        check(*part, at::kLong, "part");
        check(*counters, at::kInt, "counters");
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(logits.device());
    call(esp_argmax(logits.data_ptr(), logits.stride(0), logits.size(0), logits.size(1), dtype_code(logits),
                    mptr<int32_t>(ids), part.has_value() ? mptr<int64_t>(*part) : nullptr,
                    part.has_value() ? part->numel() : 0, counters.has_value() ? mptr<int32_t>(*counters) : nullptr,
                    counters.has_value() ? counters->numel() : 0, cur_stream()));
}

// several dense launches as one (esp_dense_multi; no reference counterpart): per group its input rows, matrices,
// output columns and plan; after[g] != 0 when group g's x is a view of group g - 1's y. The optional norm (h, d1, d2,
// w, h_out, eps) makes group 0's input RMSNorm(h + d1 + d2) * w, as dense_rmsnorm does.
void dense_multi(const std::vector<at::Tensor>& xs, const std::vector<std::vector<at::Tensor>>& T,
                 const std::vector<std::vector<at::Tensor>>& suh, const std::vector<std::vector<at::Tensor>>& svh,
                 const std::vector<std::vector<int64_t>>& col0, const std::vector<at::Tensor>& ys,
                 const std::vector<int64_t>& k2, const std::vector<int64_t>& cb, const std::vector<int64_t>& SK,
                 const std::vector<int64_t>& after, at::Tensor Z, at::Tensor counters, int64_t W, int64_t rot_smem,
                 const c10::optional<at::Tensor>& norm_h, const c10::optional<at::Tensor>& norm_d1,
                 const c10::optional<at::Tensor>& norm_d2, const c10::optional<at::Tensor>& norm_w,
                 const c10::optional<at::Tensor>& norm_h_out, double eps) {
    const size_t n = xs.size();
    TORCH_CHECK(n >= 1 && n <= 4, "dense_multi: 1 to 4 groups");
    TORCH_CHECK(T.size() == n && suh.size() == n && svh.size() == n && col0.size() == n && ys.size() == n &&
                    k2.size() == n && cb.size() == n && SK.size() == n && after.size() == n,
                "dense_multi: one entry a group in every list");
    check(Z, at::kFloat, "Z");
    check(counters, at::kInt, "counters");
    std::vector<esp_dense_group> g(n);
    const int64_t M = xs[0].size(0);
    for (size_t i = 0; i < n; ++i) {
        const at::Tensor& x = xs[i];
        const at::Tensor& y = ys[i];
        TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.stride(1) == 1 && x.size(0) == M, "x: CUDA [M, K], unit column stride");
        TORCH_CHECK(y.is_cuda() && y.dim() == 2 && y.stride(1) == 1 && y.size(0) == M, "y: CUDA [M, N], unit column stride");
        TORCH_CHECK(T[i].size() >= 1 && T[i].size() <= 4 && suh[i].size() == T[i].size() && svh[i].size() == T[i].size() &&
                        col0[i].size() == T[i].size(),
                    "dense_multi: 1 to 4 matrices a group, one entry a matrix");
        esp_dense_group& G = g[i];
        G = esp_dense_group{};
        G.x = x.data_ptr();
        G.x_dtype = dtype_code(x);
        G.x_stride = x.stride(0);
        G.K = x.size(1);
        G.n_shards = (int64_t)T[i].size();
        for (size_t s = 0; s < T[i].size(); ++s) {
            TORCH_CHECK(T[i][s].is_cuda() && T[i][s].scalar_type() == at::kShort && T[i][s].is_contiguous() &&
                            T[i][s].dim() == 3 && T[i][s].size(0) * 16 == G.K && T[i][s].size(1) * 16 == svh[i][s].numel() &&
                            T[i][s].size(2) == 8 * k2[i],
                        "trellis: contiguous int16 [K/16, N/16, 16K] matching x and svh");
            check(suh[i][s], at::kHalf, "suh");
            check(svh[i][s], at::kHalf, "svh");
            TORCH_CHECK(suh[i][s].numel() == G.K, "suh must have K elements");
            G.trellis[s] = T[i][s].data_ptr();
            G.suh[s] = suh[i][s].data_ptr();
            G.svh[s] = svh[i][s].data_ptr();
            G.n_cols[s] = svh[i][s].numel();
            G.col0[s] = col0[i][s];
        }
        G.y = y.data_ptr();
        G.y_dtype = dtype_code(y);
        G.y_stride = y.stride(0);
        G.y_cols = y.size(1);
        G.k2 = k2[i];
        G.cb = cb[i];
        G.SK = SK[i];
        G.after_previous = after[i] ? 1 : 0;
    }
    if (norm_h.has_value()) {
        const auto t = norm_h->scalar_type();
        TORCH_CHECK(norm_h->is_contiguous() && norm_w.has_value() && norm_h_out.has_value() && norm_w->scalar_type() == t &&
                        norm_h_out->scalar_type() == t && norm_h->sizes() == xs[0].sizes(),
                    "dense_multi: the norm's h, w, h_out in x's shape and dtype");
        for (const auto* d : {&norm_d1, &norm_d2})
            if (d->has_value()) TORCH_CHECK((*d)->is_contiguous() && (*d)->scalar_type() == t && (*d)->sizes() == norm_h->sizes(),
                                            "deltas: h's dtype and shape, contiguous");
        g[0].x = norm_h->data_ptr();
        g[0].x_stride = norm_h->stride(0);
        g[0].norm_h = norm_h->data_ptr();
        g[0].norm_d1 = norm_d1.has_value() ? norm_d1->data_ptr() : nullptr;
        g[0].norm_d2 = norm_d2.has_value() ? norm_d2->data_ptr() : nullptr;
        g[0].norm_w = norm_w->data_ptr();
        g[0].norm_h_out = norm_h_out->data_ptr();
        g[0].norm_eps = eps;
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(xs[0].device());
    call(esp_dense_multi((int64_t)n, g.data(), M, W, mptr<float>(Z), Z.numel(), mptr<int32_t>(counters),
                         counters.numel(), rot_smem, cur_stream()));
}

// the device status word of the current GPU (esp_status; no reference counterpart), cleared after the read if asked
int64_t status(bool clear) {
    int32_t v = 0;
    call(esp_status(&v, clear ? 1 : 0, cur_stream()));
    return v;
}

PYBIND11_MODULE(espalier_ext, m) {
    m.def("had", &had);
    m.def("route_group", &route_group);
    m.def("route_rows", &route_rows);
    m.def("dense_tile", &dense_tile);
    m.def("dense", &dense);
    m.def("group_shared", &group_shared);
    m.def("down_combine2", &down_combine2);
    m.def("grouped", &grouped);
    m.def("tile_list", &tile_list);
    m.def("grouped_list", &grouped_list);
    m.def("dequant", &dequant);
    m.def("group", &group);
    m.def("rot_in", &rot_in);
    m.def("gateup_epilogue", &gateup_epilogue);
    m.def("down_epilogue", &down_epilogue);
    m.def("combine", &combine);
    m.def("down_combine", &down_combine);
    m.def("moe_gateup", &moe_gateup);
    m.def("moe_chain", &moe_chain);
    m.def("dense_rmsnorm", &dense_rmsnorm);
    m.def("status", &status, py::arg("clear") = false);
    m.def("dense_multi", &dense_multi, py::arg("xs"), py::arg("T"), py::arg("suh"), py::arg("svh"), py::arg("col0"),
          py::arg("ys"), py::arg("k2"), py::arg("cb"), py::arg("SK"), py::arg("after"), py::arg("Z"),
          py::arg("counters"), py::arg("W"), py::arg("rot_smem"), py::arg("norm_h") = py::none(),
          py::arg("norm_d1") = py::none(), py::arg("norm_d2") = py::none(), py::arg("norm_w") = py::none(),
          py::arg("norm_h_out") = py::none(), py::arg("eps") = 0.0);
    m.def("route_group_rmsnorm", &route_group_rmsnorm);
    m.def("route_group_own", &route_group_own);
    m.def("dense_own", &dense_own);
    m.def("embed", &embed);
    m.def("add_rmsnorm", &add_rmsnorm);
    m.def("argmax", &argmax, py::arg("logits"), py::arg("ids"), py::arg("part") = py::none(),
          py::arg("counters") = py::none());
}
