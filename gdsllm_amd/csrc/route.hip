// On-device MoE routing and the MoE output epilogue.
//
// The reference routes a Qwen-MoE token on the host side of a sync: router
// logits by F.linear on the fp16 router matrix, torch.topk, a float32 softmax
// of the k logits cast back to fp16, then .tolist() of the picks
// (runtime/qwen_moe.py:386-416); after the experts it adds the shared expert
// scaled by sigmoid(shared_expert_gate . x) and clamps to the fp16 range
// (runtime/qwen_moe.py:496-513).  These kernels keep all of it on the device:
//  * gemv_f16: y = fp16(sum_k w[r][k] * x[k]) for fp16 weights (the router
//    and the shared-expert gate; the converter stores unquantized tensors as
//    fp16, tools/convert_qwen_moe.py:177-189), fp32 accumulation, each row in
//    the fixed four-part order of f16_row_dot (common.h);
//  * route_topk: the k largest logits per token in descending order (ties:
//    lower expert index first; NaN above every number, as torch.topk), and
//    fp16(softmax_fp32(those logits));
//  * moe_combine: y = clamp(expert_out + fp16(fp16(sigmoid(gate)) * shared_out))
//    with torch's fp16 elementwise semantics (each op in fp32, rounded to fp16).

#include <algorithm>

#include "common.h"
#include "topk.h"

namespace gdsllm {
namespace {

constexpr int kF16Waves = 4;      // waves per workgroup of the fp16 GEMV
constexpr int kMaxBatch = 8;
constexpr int kMaxExperts = 4096;  // 64 pick words per lane
constexpr int kMaxTopK = 64;       // one pick per lane

// Vector path (K % 8 == 0, rows and x 16-byte aligned): a 4-wave workgroup
// per row, rows dealt round-robin over the grid; wave w computes part w of
// the row (chunks w, w+4, ... of 512 columns: all its NJ loads in flight
// before the first dot product), the four wave sums meet in LDS and wave 0
// adds them in part order.  The sums are f16_row_dot's, bit for bit.
template <int NJ>
__device__ __forceinline__ void f16_row_parts(const uint16_t* __restrict__ wr, const uint16_t* __restrict__ X, int K,
                                              int nb, int64_t ldx, int wave, int lane, float (*part)[kMaxBatch]) {
    if constexpr (NJ == 0) {  // rows past 16 chunks: a loop over the part's chunks
        float acc[kMaxBatch];
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) acc[b] = 0.f;
        for (int c = 8 * lane + 512 * wave; c < K; c += 2048) {
            const uint4 w = load_nt16(wr + c);
#pragma unroll
            for (int b = 0; b < kMaxBatch; ++b) {
                if (b < nb) {
                    const uint4 xv = *reinterpret_cast<const uint4*>(X + b * ldx + c);
                    acc[b] = dot2(w.x, xv.x, acc[b]);
                    acc[b] = dot2(w.y, xv.y, acc[b]);
                    acc[b] = dot2(w.z, xv.z, acc[b]);
                    acc[b] = dot2(w.w, xv.w, acc[b]);
                }
            }
        }
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            if (b < nb) {
                const float s = group_sum<64>(acc[b]);
                if (lane == 0) part[wave][b] = s;
            }
        }
        return;
    }
    constexpr int NW = NJ > 0 ? NJ : 1;
    uint4 w[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const int c = 8 * lane + 512 * (wave + 4 * j);
        w[j] = c < K ? load_nt16(wr + c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int b = 0; b < kMaxBatch; ++b) {
        if (b < nb) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < NW; ++j) {
                const int c = 8 * lane + 512 * (wave + 4 * j);
                if (c < K) {
                    const uint4 xv = *reinterpret_cast<const uint4*>(X + b * ldx + c);
                    acc = dot2(w[j].x, xv.x, acc);
                    acc = dot2(w[j].y, xv.y, acc);
                    acc = dot2(w[j].z, xv.z, acc);
                    acc = dot2(w[j].w, xv.w, acc);
                }
            }
            const float s = group_sum<64>(acc);
            if (lane == 0) part[wave][b] = s;
        }
    }
}

// Rows blockIdx.x, += gridDim.x: y[b][r] = fp16(((p0 + p1) + p2) + p3).
template <int NJ>
__global__ __launch_bounds__(kF16Waves * 64) void gemv_f16(const uint16_t* __restrict__ W,
                                                           const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
                                                           int M, int K, int nb, int64_t ldx, int64_t ldy) {
    __shared__ float part[4][kMaxBatch];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int r = blockIdx.x; r < M; r += gridDim.x) {
        f16_row_parts<NJ>(W + static_cast<int64_t>(r) * K, X, K, nb, ldx, wave, lane, part);
        __syncthreads();
        if (wave == 0 && lane < nb)
            Y[lane * ldy + r] = f2h_bits(((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]);
        __syncthreads();
    }
}

// Scalar path (rows or x off the 16-byte grid, or K % 8 != 0): one wave per
// row, one element per lane per 64 columns.
__global__ __launch_bounds__(kF16Waves * 64) void gemv_f16_scalar(const uint16_t* __restrict__ W,
                                                                  const uint16_t* __restrict__ X,
                                                                  uint16_t* __restrict__ Y, int M, int K, int nb,
                                                                  int64_t ldx, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int wpb = static_cast<int>(blockDim.x) >> 6;
    const int nwaves = static_cast<int>(gridDim.x) * wpb;
    for (int r = static_cast<int>(blockIdx.x) * wpb + (threadIdx.x >> 6); r < M; r += nwaves) {
        const uint16_t* wr = W + static_cast<int64_t>(r) * K;
        float acc[kMaxBatch];
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) acc[b] = 0.f;
        for (int c = lane; c < K; c += 64) {
            const float w = h2f(wr[c]);
#pragma unroll
            for (int b = 0; b < kMaxBatch; ++b)
                if (b < nb) acc[b] = fmaf(w, h2f(X[b * ldx + c]), acc[b]);
        }
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            if (b < nb) {
                const float s = group_sum<64>(acc[b]);
                if (lane == 0) Y[b * ldy + r] = f2h_bits(s);
            }
        }
    }
}

// Top-k of one token by one wave.  NPL pick words per lane live in registers
// (logit lane + 64*j), NPL * 64 >= E (topk.h).
template <int NPL>
__device__ __forceinline__ void topk_wave(const uint16_t* __restrict__ L, int E, int k, int32_t* __restrict__ idx,
                                          uint16_t* __restrict__ wts, int lane) {
    // all loads first (unconditional, past E re-reading logit 0): a load under
    // a branch would be waited for before the next one is issued
    uint32_t h[NPL], word[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) h[j] = L[lane + 64 * j < E ? lane + 64 * j : 0];
#pragma unroll
    for (int j = 0; j < NPL; ++j) word[j] = lane + 64 * j < E ? pick_word(h[j], lane + 64 * j) : 0u;
    int my_idx;
    uint32_t my_key, top_key;
    topk_select<NPL>(word, k, lane, my_idx, my_key, top_key);
    const uint16_t w = topk_weight(my_key, top_key, k, lane);
    if (lane < k) {
        idx[lane] = my_idx;
        wts[lane] = w;
    }
}

// One wave per token.
template <int NPL>
__global__ __launch_bounds__(64) void route_topk(const uint16_t* __restrict__ logits, int E, int64_t ld, int k,
                                                int32_t* __restrict__ idx, uint16_t* __restrict__ wts) {
    const int64_t t = blockIdx.x;
    topk_wave<NPL>(logits + t * ld, E, k, idx + t * k, wts + t * k, static_cast<int>(threadIdx.x));
}

// y = clamp(e + fp16(fp16(sigmoid(g)) * s), -65504, 65504) elementwise, g per token.
__global__ __launch_bounds__(256) void moe_combine(const uint16_t* __restrict__ eo, const uint16_t* __restrict__ so,
                                                   const uint16_t* __restrict__ gl, uint16_t* __restrict__ y,
                                                   int64_t H, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float g = h2f(gl[i / H]);
    const float sw = h2f(f2h_bits(fp32_rounded(1.0f / fp32_rounded(1.0f + expf(-g)))));
    const float s = h2f(f2h_bits(fp32_rounded(sw * h2f(so[i]))));
    float r = h2f(f2h_bits(fp32_rounded(h2f(eo[i]) + s)));
    if (r > 65504.0f) r = 65504.0f;   // NaN compares false both ways and stays NaN
    if (r < -65504.0f) r = -65504.0f;
    y[i] = f2h_bits(r);
}

}  // namespace
}  // namespace gdsllm

using namespace gdsllm;

extern "C" int gdsllm_gemv_f16(const void* weight, const void* x, void* y, int64_t out_dim, int64_t in_dim,
                               int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    const std::string n = "gemv_f16";
    if (out_dim < 0 || in_dim < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (batch < 1 || batch > kMaxBatch)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": batch must be in [1, 8], got " + std::to_string(batch));
    if (out_dim > (int64_t(1) << 30) || in_dim > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    if (out_dim == 0 || in_dim == 0) return ok();
    if (!weight || !x || !y) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (batch > 1 && (ldx < in_dim || ldy < out_dim))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than the row length");
    if (reinterpret_cast<uintptr_t>(weight) % 2 || reinterpret_cast<uintptr_t>(x) % 2 ||
        reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": weight, x and y must be 2-byte aligned");
    const int M = static_cast<int>(out_dim), K = static_cast<int>(in_dim), B = static_cast<int>(batch);
    const bool vec = K % 8 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(x) % 16 == 0 && (B == 1 || ldx % 8 == 0);
    const auto* w = static_cast<const uint16_t*>(weight);
    const auto* xp = static_cast<const uint16_t*>(x);
    auto* yp = static_cast<uint16_t*>(y);
    const hipStream_t st = as_stream(stream);
    if (vec) {
        // a 4-wave workgroup per row (one row each while the grid fits)
        const int grid = std::min(M, 16 * cu_count());
        const int nj = ((K + 511) / 512 + 3) / 4;
        auto launch = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(grid), dim3(kF16Waves * 64), 0, st, w, xp, yp, M, K, B, ldx, ldy);
        };
        if (nj <= 1) launch(gemv_f16<1>);
        else if (nj <= 2) launch(gemv_f16<2>);
        else if (nj <= 4) launch(gemv_f16<4>);
        else launch(gemv_f16<0>);
    } else {
        const int grid = std::min((M + kF16Waves - 1) / kF16Waves, 8 * cu_count());
        hipLaunchKernelGGL(gemv_f16_scalar, dim3(grid), dim3(kF16Waves * 64), 0, st, w, xp, yp, M, K, B, ldx, ldy);
    }
    if (int rc = check_hip(hipGetLastError(), "gemv_f16 launch")) return rc;
    return ok();
}

extern "C" int gdsllm_moe_route_topk(const void* logits, int64_t num_experts, int64_t n_tok, int64_t ld_logits,
                                     int64_t top_k, int32_t* idx, void* weights, void* stream) {
    const std::string n = "moe_route_topk";
    if (num_experts < 1 || num_experts > kMaxExperts)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         n + ": num_experts must be in [1, 4096], got " + std::to_string(num_experts));
    if (top_k < 1 || top_k > kMaxTopK || top_k > num_experts)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         n + ": top_k must be in [1, min(64, num_experts)], got " + std::to_string(top_k));
    if (n_tok < 0 || n_tok > (int64_t(1) << 31) - 1)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": bad token count");
    if (n_tok == 0) return ok();
    if (ld_logits < num_experts) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ld_logits < num_experts");
    if (!logits || !idx || !weights) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (reinterpret_cast<uintptr_t>(logits) % 2 || reinterpret_cast<uintptr_t>(weights) % 2 ||
        reinterpret_cast<uintptr_t>(idx) % 4)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": misaligned pointer");
    const auto* l = static_cast<const uint16_t*>(logits);
    auto* w = static_cast<uint16_t*>(weights);
    const int E = static_cast<int>(num_experts), k = static_cast<int>(top_k);
    const dim3 grid(static_cast<unsigned>(n_tok)), block(64);
    const hipStream_t s = as_stream(stream);
    if (E <= 128) hipLaunchKernelGGL(route_topk<2>, grid, block, 0, s, l, E, ld_logits, k, idx, w);
    else if (E <= 512) hipLaunchKernelGGL(route_topk<8>, grid, block, 0, s, l, E, ld_logits, k, idx, w);
    else if (E <= 1024) hipLaunchKernelGGL(route_topk<16>, grid, block, 0, s, l, E, ld_logits, k, idx, w);
    else hipLaunchKernelGGL(route_topk<64>, grid, block, 0, s, l, E, ld_logits, k, idx, w);
    if (int rc = check_hip(hipGetLastError(), "moe_route_topk launch")) return rc;
    return ok();
}

extern "C" int gdsllm_moe_combine(const void* expert_out, const void* shared_out, const void* shared_gate_logit,
                                  void* y, int64_t hidden, int64_t n_tok, void* stream) {
    const std::string n = "moe_combine";
    if (hidden < 0 || n_tok < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (hidden > (int64_t(1) << 24) || n_tok > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    if (hidden == 0 || n_tok == 0) return ok();
    if (!expert_out || !shared_out || !shared_gate_logit || !y)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if ((reinterpret_cast<uintptr_t>(expert_out) | reinterpret_cast<uintptr_t>(shared_out) |
         reinterpret_cast<uintptr_t>(shared_gate_logit) | reinterpret_cast<uintptr_t>(y)) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": pointers must be 2-byte aligned");
    const int64_t total = hidden * n_tok;
    hipLaunchKernelGGL(moe_combine, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, as_stream(stream),
                       static_cast<const uint16_t*>(expert_out), static_cast<const uint16_t*>(shared_out),
                       static_cast<const uint16_t*>(shared_gate_logit), static_cast<uint16_t*>(y), hidden, total);
    if (int rc = check_hip(hipGetLastError(), "moe_combine launch")) return rc;
    return ok();
}
