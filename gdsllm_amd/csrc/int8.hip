// Per-column int8 weights: the converter's "int8" format (tools/
// convert_weights.py:55-83: W_int8 [out, in], scale fp16 [1, in]) and the
// projection the reference computes from it in runtime/llama.py:162-165,
// w = (w.float() * scale).half(); F.linear(x, w).
//
// Every weight is rebuilt in registers as exactly the reference's fp16 value
// RN16(q * s): the biased byte becomes the fp16 number 1152 + q through one
// v_perm (0x64 high byte over q ^ 0x80: 1024 + 128 + q), minus 1152 is exact,
// and the packed multiply by s rounds the exact product q * s once.  The
// products with x are then summed in fp32 (v_dot2_f32_f16), so the GEMV
// differs from the reference's F.linear only in summation order, and the
// dequant kernel is bit-exact.

#include <algorithm>

#include "common.h"

namespace gdsllm {
namespace {

constexpr int kI8Threads = 256;
constexpr int kI8Waves = kI8Threads / 64;
constexpr int kI8Rows = 4;  // rows per wave

// fp16 pairs (1152 + q0, 1152 + q1) and (1152 + q2, 1152 + q3) of the four
// signed bytes of w: v_perm places 0x64 over each biased byte.
__device__ __forceinline__ void i8_codes(uint32_t w, uint32_t& c01, uint32_t& c23) {
    const uint32_t u = w ^ 0x80808080u;
    c01 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    c23 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}

// RN16(q * s) for a pair: (1152 + q) - 1152 is exact in fp16, the product
// rounds once.
__device__ __forceinline__ half2_t i8_weights(uint32_t codes, uint32_t s) {
    const half2_t off = {static_cast<half_t>(-1152.0f), static_cast<half_t>(-1152.0f)};
    return (__builtin_bit_cast(half2_t, codes) + off) * __builtin_bit_cast(half2_t, s);
}

// Bit-exact fp16 weights: thread t converts 16 consecutive weights of a row.
__global__ __launch_bounds__(kI8Threads) void int8_dequant16(const int8_t* __restrict__ W,
                                                             const uint16_t* __restrict__ S, uint4* __restrict__ out,
                                                             int64_t chunks, int cpr) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kI8Threads) + threadIdx.x; i < chunks;
         i += static_cast<int64_t>(gridDim.x) * kI8Threads) {
        const int c = static_cast<int>(i % cpr);
        const uint4 w = load_nt16(W + 16 * i);
        const uint4 s0 = *reinterpret_cast<const uint4*>(S + 16 * c);
        const uint4 s1 = *reinterpret_cast<const uint4*>(S + 16 * c + 8);
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
        const uint32_t sd[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        uint32_t o[8];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t c01, c23;
            i8_codes(wd[d], c01, c23);
            o[2 * d] = __builtin_bit_cast(uint32_t, i8_weights(c01, sd[2 * d]));
            o[2 * d + 1] = __builtin_bit_cast(uint32_t, i8_weights(c23, sd[2 * d + 1]));
        }
        out[2 * i] = make_uint4(o[0], o[1], o[2], o[3]);
        out[2 * i + 1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
}

// Any shape and alignment: one thread per element, the reference's order.
__global__ __launch_bounds__(kI8Threads) void int8_dequant_elems(const int8_t* __restrict__ W,
                                                                 const uint16_t* __restrict__ S,
                                                                 uint16_t* __restrict__ out, int64_t n, int64_t cols) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kI8Threads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kI8Threads) {
        const float v = fp32_rounded(static_cast<float>(W[i]) * h2f(S[i % cols]));
        out[i] = f2h_bits(v);
    }
}

// Sums acc[0..3] over the wave; lane L receives the total of entry L >> 4.
__device__ __forceinline__ float i8_reduce4(const float (&acc)[4]) {
    const float k02 = swap_sum32(acc[0], acc[2]);
    const float k13 = swap_sum32(acc[1], acc[3]);
    return row16_sum(swap_sum16(k02, k13));
}

// y[b][r] = sum_k RN16(q[r][k] * s[k]) * x[b][k], fp32 accumulation.  A wave
// owns kI8Rows rows at a time; lane l walks 16-byte chunks l, l + 64, ... of
// them with the next chunk's loads in flight while it computes the current
// one.  Needs in_dim % 16 == 0 and 16-byte aligned W, S and x rows.  Rows past
// M read row M - 1, batch rows past nb read row nb - 1; neither is stored.
template <int NB>
__global__ __launch_bounds__(kI8Threads) void int8_gemv(const int8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                                        const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
                                                        int M, int K, int nb, int64_t ldx, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * kI8Waves + (threadIdx.x >> 6);
    const int nw = gridDim.x * kI8Waves;
    const int cpr = K >> 4;
    const uint16_t* xr[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) xr[b] = X + static_cast<int64_t>(b < nb ? b : nb - 1) * ldx;

    struct Chunk {
        uint4 w[kI8Rows];
        uint4 s[2];
        uint4 x[NB][2];
    };
    for (int r0 = gw * kI8Rows; r0 < M; r0 += nw * kI8Rows) {
        const int8_t* wr[kI8Rows];
#pragma unroll
        for (int i = 0; i < kI8Rows; ++i) wr[i] = W + static_cast<int64_t>(min(r0 + i, M - 1)) * K;
        auto load = [&](int c, Chunk& ch) {
#pragma unroll
            for (int i = 0; i < kI8Rows; ++i) ch.w[i] = load_nt16(wr[i] + 16 * c);
            ch.s[0] = *reinterpret_cast<const uint4*>(S + 16 * c);
            ch.s[1] = *reinterpret_cast<const uint4*>(S + 16 * c + 8);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                ch.x[b][0] = *reinterpret_cast<const uint4*>(xr[b] + 16 * c);
                ch.x[b][1] = *reinterpret_cast<const uint4*>(xr[b] + 16 * c + 8);
            }
        };
        float acc[NB][kI8Rows];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < kI8Rows; ++i) acc[b][i] = 0.f;
        auto compute = [&](const Chunk& ch) {
            const uint32_t sd[8] = {ch.s[0].x, ch.s[0].y, ch.s[0].z, ch.s[0].w,
                                    ch.s[1].x, ch.s[1].y, ch.s[1].z, ch.s[1].w};
#pragma unroll
            for (int i = 0; i < kI8Rows; ++i) {
                const uint32_t wd[4] = {ch.w[i].x, ch.w[i].y, ch.w[i].z, ch.w[i].w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    uint32_t c01, c23;
                    i8_codes(wd[d], c01, c23);
                    const uint32_t w01 = __builtin_bit_cast(uint32_t, i8_weights(c01, sd[2 * d]));
                    const uint32_t w23 = __builtin_bit_cast(uint32_t, i8_weights(c23, sd[2 * d + 1]));
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const uint32_t xd[8] = {ch.x[b][0].x, ch.x[b][0].y, ch.x[b][0].z, ch.x[b][0].w,
                                                ch.x[b][1].x, ch.x[b][1].y, ch.x[b][1].z, ch.x[b][1].w};
                        acc[b][i] = dot2(w01, xd[2 * d], acc[b][i]);
                        acc[b][i] = dot2(w23, xd[2 * d + 1], acc[b][i]);
                    }
                }
            }
        };
        if (lane < cpr) {
            Chunk cur, nxt;
            load(lane, cur);
            int c = lane;
            for (; c + 64 < cpr; c += 64) {
                load(c + 64, nxt);
                compute(cur);
                cur = nxt;
            }
            compute(cur);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float v = i8_reduce4(acc[b]);
            const int r = r0 + (lane >> 4);
            if ((lane & 15) == 0 && b < nb && r < M) Y[b * ldy + r] = f2h_bits(v);
        }
    }
}

// Any in_dim and alignment: one wave per row, lanes stride over elements.
__global__ __launch_bounds__(kI8Threads) void int8_gemv_generic(const int8_t* __restrict__ W,
                                                                const uint16_t* __restrict__ S,
                                                                const uint16_t* __restrict__ X,
                                                                uint16_t* __restrict__ Y, int M, int K, int nb,
                                                                int64_t ldx, int64_t ldy) {
    const int row = blockIdx.x * kI8Waves + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int8_t* wr = W + static_cast<int64_t>(row) * K;
    for (int b = 0; b < nb; ++b) {
        float acc = 0.f;
        for (int k = lane; k < K; k += 64) {
            const float w = h2f(f2h_bits(fp32_rounded(static_cast<float>(wr[k]) * h2f(S[k]))));
            acc = __builtin_fmaf(w, h2f(X[b * ldx + k]), acc);
        }
        acc = group_sum<64>(acc);
        if (lane == 0) Y[b * ldy + row] = f2h_bits(acc);
    }
}

int grid_for(int64_t items, int per_block) {
    const int64_t cap = static_cast<int64_t>(cu_count()) * 16;
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((items + per_block - 1) / per_block, cap)));
}

template <int NB>
void launch_int8_gemv(const int8_t* w, const uint16_t* s, const uint16_t* x, uint16_t* y, int M, int K, int nb,
                      int64_t ldx, int64_t ldy, hipStream_t st) {
    const int groups = (M + kI8Rows - 1) / kI8Rows;
    hipLaunchKernelGGL(int8_gemv<NB>, dim3(grid_for(groups, kI8Waves)), dim3(kI8Threads), 0, st, w, s, x, y, M, K,
                       nb, ldx, ldy);
}

}  // namespace

extern "C" int gdsllm_dequant_int8(const void* weight, const void* scale, void* dst, int64_t rows, int64_t cols,
                                   void* stream) {
    if (rows < 0 || cols < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_int8: negative dimension");
    if (rows == 0 || cols == 0) return ok();
    if (!weight || !scale || !dst) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_int8: null pointer");
    if (rows > (int64_t(1) << 31) || cols > (int64_t(1) << 31))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_int8: dimension too large");
    if (reinterpret_cast<uintptr_t>(scale) % 2 || reinterpret_cast<uintptr_t>(dst) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_int8: scale and dst must be 2-byte aligned");
    hipStream_t s = as_stream(stream);
    const bool fast = cols % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(scale) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0;
    if (fast) {
        const int64_t chunks = rows * cols / 16;
        hipLaunchKernelGGL(int8_dequant16, dim3(grid_for(chunks, kI8Threads)), dim3(kI8Threads), 0, s,
                           static_cast<const int8_t*>(weight), static_cast<const uint16_t*>(scale),
                           static_cast<uint4*>(dst), chunks, static_cast<int>(cols / 16));
    } else {
        hipLaunchKernelGGL(int8_dequant_elems, dim3(grid_for(rows * cols, kI8Threads)), dim3(kI8Threads), 0, s,
                           static_cast<const int8_t*>(weight), static_cast<const uint16_t*>(scale),
                           static_cast<uint16_t*>(dst), rows * cols, cols);
    }
    if (int rc = check_hip(hipGetLastError(), "dequant_int8 launch")) return rc;
    return ok();
}

extern "C" int gdsllm_fused_int8_gemv(const void* weight, const void* scale, const void* x, void* y, int64_t out_dim,
                                      int64_t in_dim, int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    const std::string n = "fused_int8_gemv";
    if (out_dim < 0 || in_dim < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (batch < 1 || batch > 8)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": batch must be in [1, 8], got " + std::to_string(batch));
    if (out_dim > (int64_t(1) << 30) || in_dim > (int64_t(1) << 30))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    if (out_dim == 0 || in_dim == 0) return ok();
    if (!weight || !scale || !x || !y) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (batch > 1 && (ldx < in_dim || ldy < out_dim))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than the row length");
    if (reinterpret_cast<uintptr_t>(scale) % 2 || reinterpret_cast<uintptr_t>(x) % 2 ||
        reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": scale, x and y must be 2-byte aligned");
    hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(out_dim), K = static_cast<int>(in_dim), nb = static_cast<int>(batch);
    const auto* w = static_cast<const int8_t*>(weight);
    const auto* sc = static_cast<const uint16_t*>(scale);
    const auto* xp = static_cast<const uint16_t*>(x);
    auto* yp = static_cast<uint16_t*>(y);
    const bool fast = K % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(scale) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                      (nb == 1 || ldx % 8 == 0);
    if (fast) {
        if (nb == 1)
            launch_int8_gemv<1>(w, sc, xp, yp, M, K, nb, ldx, ldy, s);
        else if (nb == 2)
            launch_int8_gemv<2>(w, sc, xp, yp, M, K, nb, ldx, ldy, s);
        else if (nb <= 4)
            launch_int8_gemv<4>(w, sc, xp, yp, M, K, nb, ldx, ldy, s);
        else
            launch_int8_gemv<8>(w, sc, xp, yp, M, K, nb, ldx, ldy, s);
    } else {
        hipLaunchKernelGGL(int8_gemv_generic, dim3((M + kI8Waves - 1) / kI8Waves), dim3(kI8Threads), 0, s, w, sc, xp,
                           yp, M, K, nb, ldx, ldy);
    }
    if (int rc = check_hip(hipGetLastError(), "fused_int8_gemv launch")) return rc;
    return ok();
}

}  // namespace gdsllm
