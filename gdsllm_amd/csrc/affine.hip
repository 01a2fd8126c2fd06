// Affine-Q4 (SWAN / Qwen-MoE) fused dequant + GEMV, and the top-k expert
// gather MLP built from it, for gfx950.
//
// GEMV semantics follow kernel_fused_affine_q4_gemv
// (runtime/affine_q4_dequant.cu:79-158): y[r] = fp16(sum_k (nib*s_G + b_G)*x[k]),
// fp32 accumulation.  The gather MLP reproduces the decode branch of
// moe_mlp_selective (runtime/qwen_moe.py:455-474): per selected expert,
// gate/up GEMVs rounded to fp16, h = fp16(fp16(silu(gate)) * up), the down GEMV,
// and the routing-weighted sum (accumulated in fp32 here, rounded once).
//
// Layout: words [rows][in_dim/8], nibble n of a word = element 8w+n (LSB first);
// fp16 scale/bias [rows][in_dim/g].  A 16-byte chunk = 4 words = 32 elements,
// always inside one group when g % 32 == 0, so a lane's unit of work is one
// chunk: a single coalesced 16-byte load (no re-blocking needed, unlike the
// 18-byte GGUF blocks).  Nibble pairs become fp16 with the exponent trick
// ((q|0x6400) = 1024+q, (q<<4|0x5400) = 64+q) and feed v_dot2_f32_f16 against
// an LDS copy of x pre-permuted into the same pair order, with per-chunk
// corrections, so chunk = s*(S - corr) + b*sum(x).
//
// Gather MLP = two launches.  Phase 1 treats the 2*top_k*ffn selected gate/up
// rows as one virtual matrix (expert rows located by index on device) and
// writes their fp16 outputs to the workspace.  Phase 2 builds h for every
// selected expert into LDS and computes each output row as the weighted sum
// over experts of the down-projection rows.

#include <mutex>
#include <utility>
#include <vector>

#include "common.h"

namespace gdsllm {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// Prepared-x record per 32-element chunk: 16 packed pairs (64 B), fp32
// correction, fp32 sum, 8 B pad.  80 B = 4*5 dwords: consecutive records sit
// on distinct banks for ds_read_b128.
constexpr int kRec = 80;
constexpr int kU = 8;  // chunk loads in flight per lane

// Pairs of the 8 elements of one word in the order the unpacked nibbles come
// out: (x0,x4) (x1,x5) (x2,x6) (x3,x7); `a`..`d` hold x0..x7 as packed fp16.
__device__ __forceinline__ uint4 word_pairs(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return make_uint4((a & 0xFFFFu) | (c << 16), (a >> 16) | (c & 0xFFFF0000u), (b & 0xFFFFu) | (d << 16),
                      (b >> 16) | (d & 0xFFFF0000u));
}

// Writes the record quarter (one word = 8 elements) held by this thread and the
// partial correction / sum; the caller reduces across the 4 quarter lanes.
__device__ __forceinline__ void xprep_quarter(uint8_t* rec, int wq, uint4 eight, float& corr, float& sum) {
    *reinterpret_cast<uint4*>(rec + 16 * wq) = word_pairs(eight.x, eight.y, eight.z, eight.w);
    const float x0 = h2f(eight.x & 0xFFFFu), x1 = h2f(eight.x >> 16), x2 = h2f(eight.y & 0xFFFFu),
                x3 = h2f(eight.y >> 16), x4 = h2f(eight.z & 0xFFFFu), x5 = h2f(eight.z >> 16),
                x6 = h2f(eight.w & 0xFFFFu), x7 = h2f(eight.w >> 16);
    corr = 1024.f * (x0 + x2 + x4 + x6) + 64.f * (x1 + x3 + x5 + x7);
    sum = ((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7));
}

// 8 consecutive fp16 from global memory.
__device__ __forceinline__ uint4 load8h(const uint16_t* p, bool aligned16) {
    if (aligned16) return *reinterpret_cast<const uint4*>(p);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = static_cast<uint32_t>(p[2 * i]) | (static_cast<uint32_t>(p[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Records for NB rows of x (row b at X + b*ldx), `chunks` chunks each.
template <int NB>
__device__ void build_xprep_plain(uint8_t* xp, const uint16_t* __restrict__ X, int chunks, int64_t ldx, bool al16) {
    const int items = NB * chunks * 4;
    for (int base = 0; base < items; base += kThreads) {
        const int it = base + threadIdx.x;
        const bool live = it < items;
        const int wq = it & 3;
        const int c = (it >> 2) % chunks;
        const int b = (it >> 2) / chunks;
        float corr = 0.f, sum = 0.f;
        uint8_t* rec = xp + (b * chunks + c) * kRec;
        if (live) xprep_quarter(rec, wq, load8h(X + b * ldx + 32 * c + 8 * wq, al16), corr, sum);
        corr += __shfl_xor(corr, 1, 4);
        corr += __shfl_xor(corr, 2, 4);
        sum += __shfl_xor(sum, 1, 4);
        sum += __shfl_xor(sum, 2, 4);
        if (live && wq == 0) {
            *reinterpret_cast<float*>(rec + 64) = corr;
            *reinterpret_cast<float*>(rec + 68) = sum;
        }
    }
}

// Dot of one 32-element chunk with its prepared record: s*(S - corr) + b*sum.
__device__ __forceinline__ float chunk_dot(uint4 w, const uint8_t* rec, float s, float b) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    float S = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 xv = *reinterpret_cast<const uint4*>(rec + 16 * q);
        const uint32_t v = wd[q], vs = v >> 8;
        S = dot2(nib_lo_pair(v), xv.x, S);
        S = dot2(nib_hi_pair(v), xv.y, S);
        S = dot2(nib_lo_pair(vs), xv.z, S);
        S = dot2(nib_hi_pair(vs), xv.w, S);
    }
    const float2 cs = *reinterpret_cast<const float2*>(rec + 64);
    return __builtin_fmaf(s, S - cs.x, b * cs.y);
}

// Where one row of a GEMV lives and where its result goes.
struct PlainRows {
    const uint32_t* W;
    const uint16_t* S;
    const uint16_t* B;
    uint16_t* Y;
    int64_t ldy;
    int M;
    __device__ bool locate(int row, const uint32_t*& w, const uint16_t*& s, const uint16_t*& b, int K, int gpr) const {
        w = W + static_cast<int64_t>(row) * (K / 8);
        s = S + static_cast<int64_t>(row) * gpr;
        b = B + static_cast<int64_t>(row) * gpr;
        return true;
    }
    __device__ void store(int bidx, int row, float v) const { Y[bidx * ldy + row] = f2h_bits(v); }
};

// Gate/up rows of the selected experts: row r -> slot k = r / (2F),
// projection (r / F) & 1 (0 = gate, 1 = up), expert row n = r % F.
struct GateUpRows {
    gdsllm_affine_experts gate, up;
    const int32_t* idx;
    uint16_t* out;  // fp16 [top_k][2][F]
    int F;
    int M;
    __device__ bool locate(int row, const uint32_t*& w, const uint16_t*& s, const uint16_t*& b, int K, int gpr) const {
        const int k = row / (2 * F);
        const int n = row % F;
        const gdsllm_affine_experts& p = ((row / F) & 1) ? up : gate;
        const int e = idx[k];
        if (e < 0 || e >= p.num_experts) return false;
        w = reinterpret_cast<const uint32_t*>(static_cast<const char*>(p.weight) + e * p.weight_stride) +
            static_cast<int64_t>(n) * (K / 8);
        s = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.scales) + e * p.scale_stride) +
            static_cast<int64_t>(n) * gpr;
        b = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.biases) + e * p.bias_stride) +
            static_cast<int64_t>(n) * gpr;
        return true;
    }
    __device__ void store(int, int row, float v) const { out[row] = f2h_bits(v); }
};

// Generic affine GEMV: LR lanes share a row (64/LR rows per wave pass), each
// lane walks chunks lane%LR, +LR, ... of its row; loads are issued kU items
// ahead of the math.  NB batch rows of x share every weight load.
template <int LR, int NB, class Rows>
__global__ __launch_bounds__(kThreads) void affine_gemv(Rows rows, const uint16_t* __restrict__ X, int K, int gsize,
                                                        int64_t ldx, int x_al16) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int CPR = K / 32;
    build_xprep_plain<NB>(smem, X, CPR, ldx, x_al16 != 0);
    __syncthreads();

    constexpr int RW = 64 / LR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LR, li = lane % LR;
    const int gpr = K / gsize;
    const int CPL = (CPR + LR - 1) / LR;
    const int passes = (rows.M + RW - 1) / RW;
    const int TW = gridDim.x * kWaves;
    const int gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int my_passes = gw < passes ? (passes - 1 - gw) / TW + 1 : 0;
    const int n_items = my_passes * CPL;

    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;

    for (int base = 0; base < n_items; base += kU) {
        uint4 wv[kU];
        float sv[kU], bv[kU];
        bool ok[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int it = base + u;
            const int pass = gw + (it / CPL) * TW;
            const int t = it % CPL;
            const int row = pass * RW + sub;
            const int c = li + LR * t;
            ok[u] = false;
            if (it < n_items && row < rows.M && c < CPR) {
                const uint32_t* w;
                const uint16_t *s, *b;
                if (rows.locate(row, w, s, b, K, gpr)) {
                    ok[u] = true;
                    wv[u] = load_nt16(w + 4 * c);
                    const int G = (32 * c) / gsize;
                    sv[u] = h2f(s[G]);
                    bv[u] = h2f(b[G]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int it = base + u;
            if (it >= n_items) break;
            const int t = it % CPL;
            if (ok[u]) {
                const int c = li + LR * t;
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    acc[b] += chunk_dot(wv[u], smem + (b * CPR + c) * kRec, sv[u], bv[u]);
            }
            if (t == CPL - 1) {
                const int row = (gw + (it / CPL) * TW) * RW + sub;
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const float v = group_sum<LR>(acc[b]);
                    if (li == 0 && row < rows.M) rows.store(b, row, v);
                    acc[b] = 0.f;
                }
            }
        }
    }
}

// Phase 2 of the gather MLP.  h_k = fp16(fp16(silu(g)) * u) for every selected
// expert goes into LDS as prepared records; each output row o then sums
// w_k * down[idx_k][o] . h_k over the top_k experts.
template <int LR>
__global__ __launch_bounds__(kThreads) void moe_down(gdsllm_affine_experts down, const int32_t* __restrict__ idx,
                                                     const uint16_t* __restrict__ rw,
                                                     const uint16_t* __restrict__ gu, int top_k,
                                                     uint16_t* __restrict__ Y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int F = static_cast<int>(down.in_dim);
    const int H = static_cast<int>(down.out_dim);
    const int gsize = static_cast<int>(down.group_size);
    const int CPR = F / 32;
    // prepared h records: [top_k][CPR]
    {
        const int items = top_k * CPR * 4;
        for (int base = 0; base < items; base += kThreads) {
            const int it = base + threadIdx.x;
            const bool live = it < items;
            const int wq = it & 3, c = (it >> 2) % CPR, k = (it >> 2) / CPR;
            float corr = 0.f, sum = 0.f;
            uint8_t* rec = smem + (k * CPR + c) * kRec;
            if (live) {
                const uint16_t* gp = gu + static_cast<int64_t>(k) * 2 * F + 32 * c + 8 * wq;
                const uint16_t* up = gp + F;
                uint32_t hw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint16_t h2[2];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float g = h2f(gp[2 * i + j]);
                        const float sg = h2f(f2h_bits(g / (1.0f + expf(-g))));
                        h2[j] = f2h_bits(sg * h2f(up[2 * i + j]));
                    }
                    hw[i] = static_cast<uint32_t>(h2[0]) | (static_cast<uint32_t>(h2[1]) << 16);
                }
                xprep_quarter(rec, wq, make_uint4(hw[0], hw[1], hw[2], hw[3]), corr, sum);
            }
            corr += __shfl_xor(corr, 1, 4);
            corr += __shfl_xor(corr, 2, 4);
            sum += __shfl_xor(sum, 1, 4);
            sum += __shfl_xor(sum, 2, 4);
            if (live && wq == 0) {
                *reinterpret_cast<float*>(rec + 64) = corr;
                *reinterpret_cast<float*>(rec + 68) = sum;
            }
        }
    }
    __syncthreads();

    constexpr int RW = 64 / LR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LR, li = lane % LR;
    const int gpr = F / gsize;
    const int CPL = (CPR + LR - 1) / LR;
    const int passes = (H + RW - 1) / RW;
    const int TW = gridDim.x * kWaves;
    const int gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    for (int pass = gw; pass < passes; pass += TW) {
        const int o = pass * RW + sub;
        float acc = 0.f;
        for (int t = 0; t < CPL; ++t) {
            const int c = li + LR * t;
            for (int k0 = 0; k0 < top_k; k0 += kU) {
                uint4 wv[kU];
                float sv[kU], bv[kU], wk[kU];
                bool ok[kU];
#pragma unroll
                for (int u = 0; u < kU; ++u) {
                    const int k = k0 + u;
                    ok[u] = false;
                    if (k < top_k && o < H && c < CPR) {
                        const int e = idx[k];
                        if (e >= 0 && e < down.num_experts) {
                            ok[u] = true;
                            const uint32_t* w =
                                reinterpret_cast<const uint32_t*>(static_cast<const char*>(down.weight) +
                                                                  e * down.weight_stride) +
                                static_cast<int64_t>(o) * (F / 8);
                            const uint16_t* s =
                                reinterpret_cast<const uint16_t*>(static_cast<const char*>(down.scales) +
                                                                  e * down.scale_stride) +
                                static_cast<int64_t>(o) * gpr;
                            const uint16_t* b =
                                reinterpret_cast<const uint16_t*>(static_cast<const char*>(down.biases) +
                                                                  e * down.bias_stride) +
                                static_cast<int64_t>(o) * gpr;
                            const int G = (32 * c) / gsize;
                            wv[u] = load_nt16(w + 4 * c);
                            sv[u] = h2f(s[G]);
                            bv[u] = h2f(b[G]);
                            wk[u] = h2f(rw[k]);
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < kU; ++u)
                    if (ok[u]) acc = __builtin_fmaf(wk[u], chunk_dot(wv[u], smem + ((k0 + u) * CPR + c) * kRec, sv[u], bv[u]), acc);
            }
        }
        acc = group_sum<LR>(acc);
        if (li == 0 && o < H) Y[o] = f2h_bits(acc);
    }
}

int blocks_per_cu(const void* fn, size_t lds) {
    static std::mutex mu;
    static std::vector<std::pair<std::pair<const void*, size_t>, int>> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (auto& e : cache)
        if (e.first.first == fn && e.first.second == lds) return e.second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kThreads, lds) != hipSuccess || n <= 0) n = 1;
    cache.push_back({{fn, lds}, n});
    return n;
}

int prepare(const void* fn, size_t lds) {
    if (lds > 65536)
        return check_hip(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                         "hipFuncSetAttribute");
    return GDSLLM_OK;
}

// Lanes per row: the widest power of two <= min(64, chunks per row).
int lanes_per_row(int cpr) {
    int lr = 64;
    while (lr > 8 && lr > cpr) lr >>= 1;
    return lr;
}

template <int LR, int NB, class Rows>
int launch_affine_gemv(const Rows& rows, const uint16_t* x, int K, int gsize, int64_t ldx, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(&affine_gemv<LR, NB, Rows>);
    const size_t lds = static_cast<size_t>(NB) * (K / 32) * kRec;
    if (int rc = prepare(fn, lds)) return rc;
    const int passes = (rows.M + 64 / LR - 1) / (64 / LR);
    const int need = (passes + kWaves - 1) / kWaves;
    const int cap = blocks_per_cu(fn, lds) * cu_count();
    const int grid = need < cap ? need : cap;
    const bool al16 = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (ldx % 8 == 0);
    hipLaunchKernelGGL((affine_gemv<LR, NB, Rows>), dim3(grid), dim3(kThreads), lds, stream, rows, x, K, gsize, ldx,
                       al16 ? 1 : 0);
    return check_hip(hipGetLastError(), "affine_gemv launch");
}

template <int NB, class Rows>
int dispatch_lr(const Rows& rows, const uint16_t* x, int K, int gsize, int64_t ldx, hipStream_t stream) {
    switch (lanes_per_row(K / 32)) {
        case 64: return launch_affine_gemv<64, NB>(rows, x, K, gsize, ldx, stream);
        case 32: return launch_affine_gemv<32, NB>(rows, x, K, gsize, ldx, stream);
        case 16: return launch_affine_gemv<16, NB>(rows, x, K, gsize, ldx, stream);
        default: return launch_affine_gemv<8, NB>(rows, x, K, gsize, ldx, stream);
    }
}

// Any shape with in_dim % 8 == 0 and in_dim % group_size == 0: one wave per
// row, one lane per word, the reference's per-element arithmetic.
__global__ __launch_bounds__(256) void affine_gemv_generic(const uint32_t* __restrict__ W,
                                                           const uint16_t* __restrict__ S,
                                                           const uint16_t* __restrict__ B,
                                                           const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
                                                           int M, int K, int gsize, int NB, int64_t ldx,
                                                           int64_t ldy) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int wpr = K / 8, gpr = K / gsize;
    for (int bi = 0; bi < NB; ++bi) {
        float acc = 0.f;
        for (int w = lane; w < wpr; w += 64) {
            const uint32_t v = W[static_cast<int64_t>(row) * wpr + w];
            const int G = (8 * w) / gsize;
            const float s = h2f(S[static_cast<int64_t>(row) * gpr + G]);
            const float b = h2f(B[static_cast<int64_t>(row) * gpr + G]);
            for (int n = 0; n < 8; ++n) {
                const float val = static_cast<float>((v >> (4 * n)) & 15u) * s + b;
                acc = __builtin_fmaf(val, h2f(X[bi * ldx + 8 * w + n]), acc);
            }
        }
        acc = group_sum<64>(acc);
        if (lane == 0) Y[bi * ldy + row] = f2h_bits(acc);
    }
}

}  // namespace
}  // namespace gdsllm

using namespace gdsllm;

extern "C" int gdsllm_fused_affine_q4_gemv(const void* weight, const void* scales, const void* biases, const void* x,
                                           void* y, int64_t out_dim, int64_t in_dim, int64_t group_size,
                                           int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    const std::string n = "fused_affine_q4_gemv";
    if (out_dim < 0 || in_dim < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (batch < 1 || batch > 8)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": batch must be in [1, 8], got " + std::to_string(batch));
    if (out_dim == 0 || in_dim == 0) return ok();
    if (group_size <= 0 || group_size % 8 != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": group_size must be a positive multiple of 8, got " +
                                                          std::to_string(group_size));
    if (in_dim % group_size != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": in_dim " + std::to_string(in_dim) +
                                                          " is not a multiple of group_size " +
                                                          std::to_string(group_size));
    if (!weight || !scales || !biases || !x || !y) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (out_dim > (int64_t(1) << 30) || in_dim > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    if (batch > 1 && (ldx < in_dim || ldy < out_dim))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than the row length");
    if (reinterpret_cast<uintptr_t>(weight) % 4 || reinterpret_cast<uintptr_t>(scales) % 2 ||
        reinterpret_cast<uintptr_t>(biases) % 2 || reinterpret_cast<uintptr_t>(x) % 2 ||
        reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": misaligned pointer");
    hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(out_dim), K = static_cast<int>(in_dim), g = static_cast<int>(group_size);
    const auto* xp = static_cast<const uint16_t*>(x);
    auto* yp = static_cast<uint16_t*>(y);
    const bool fast = (K % 32 == 0) && (g % 32 == 0) && (reinterpret_cast<uintptr_t>(weight) % 16 == 0);
    const size_t budget = static_cast<size_t>(max_lds_bytes());
    if (fast && static_cast<size_t>(K / 32) * kRec <= budget) {
        int64_t b0 = 0;
        while (b0 < batch) {
            int nb = 8;
            while (nb > 1 && (nb > batch - b0 || static_cast<size_t>(nb) * (K / 32) * kRec > budget)) nb >>= 1;
            PlainRows rows{static_cast<const uint32_t*>(weight), static_cast<const uint16_t*>(scales),
                           static_cast<const uint16_t*>(biases), yp + b0 * ldy, ldy, M};
            const uint16_t* xb = xp + b0 * ldx;
            int rc;
            switch (nb) {
                case 8: rc = dispatch_lr<8>(rows, xb, K, g, ldx, s); break;
                case 4: rc = dispatch_lr<4>(rows, xb, K, g, ldx, s); break;
                case 2: rc = dispatch_lr<2>(rows, xb, K, g, ldx, s); break;
                default: rc = dispatch_lr<1>(rows, xb, K, g, ldx, s); break;
            }
            if (rc) return rc;
            b0 += nb;
        }
        return ok();
    }
    hipLaunchKernelGGL(affine_gemv_generic, dim3((M + 3) / 4), dim3(256), 0, s, static_cast<const uint32_t*>(weight),
                       static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases), xp, yp, M, K, g,
                       static_cast<int>(batch), ldx, ldy);
    if (int rc = check_hip(hipGetLastError(), "affine_gemv_generic launch")) return rc;
    return ok();
}

extern "C" size_t gdsllm_moe_gather_workspace_size(int64_t top_k, int64_t ffn_dim) {
    if (top_k <= 0 || ffn_dim <= 0) return 256;
    const size_t bytes = static_cast<size_t>(top_k) * 2 * static_cast<size_t>(ffn_dim) * 2;
    return (bytes + 255) / 256 * 256;
}

static int check_experts(const gdsllm_affine_experts* p, const char* what, std::string& err) {
    if (!p) { err = std::string(what) + " is null"; return 1; }
    if (!p->weight || !p->scales || !p->biases) { err = std::string(what) + ": null pointer"; return 1; }
    if (p->num_experts <= 0 || p->out_dim <= 0 || p->in_dim <= 0 || p->group_size <= 0) {
        err = std::string(what) + ": non-positive size";
        return 1;
    }
    if (p->in_dim % 32 != 0 || p->group_size % 32 != 0 || p->in_dim % p->group_size != 0) {
        err = std::string(what) + ": in_dim and group_size must be multiples of 32 and in_dim of group_size";
        return 1;
    }
    if (p->out_dim > (int64_t(1) << 24) || p->in_dim > (int64_t(1) << 20)) {
        err = std::string(what) + ": dimension too large";
        return 1;
    }
    if (reinterpret_cast<uintptr_t>(p->weight) % 16 || p->weight_stride % 16 ||
        reinterpret_cast<uintptr_t>(p->scales) % 2 || reinterpret_cast<uintptr_t>(p->biases) % 2 ||
        p->scale_stride % 2 || p->bias_stride % 2) {
        err = std::string(what) + ": weight must be 16-byte aligned (and its expert stride), scales/biases 2-byte";
        return 1;
    }
    return 0;
}

extern "C" int gdsllm_moe_gather_affine_q4(const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                                           const gdsllm_affine_experts* down, const void* x, const int32_t* idx,
                                           const void* routing_weights, int64_t top_k, void* y, void* workspace,
                                           size_t workspace_bytes, void* stream) {
    const std::string n = "moe_gather_affine_q4";
    std::string err;
    if (check_experts(gate, "gate", err) || check_experts(up, "up", err) || check_experts(down, "down", err))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": " + err);
    if (top_k < 1 || top_k > 64)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": top_k must be in [1, 64], got " + std::to_string(top_k));
    const int64_t H = gate->in_dim, F = gate->out_dim;
    if (up->in_dim != H || up->out_dim != F || down->in_dim != F || down->out_dim != H ||
        gate->group_size != up->group_size || up->num_experts != gate->num_experts ||
        down->num_experts != gate->num_experts)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": gate/up [E,F,H] and down [E,H,F] shapes disagree");
    if (!x || !idx || !routing_weights || !y || !workspace)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 2 || reinterpret_cast<uintptr_t>(y) % 2 ||
        reinterpret_cast<uintptr_t>(routing_weights) % 2 || reinterpret_cast<uintptr_t>(idx) % 4 ||
        reinterpret_cast<uintptr_t>(workspace) % 16)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": misaligned pointer");
    if (workspace_bytes < gdsllm_moe_gather_workspace_size(top_k, F))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": workspace too small (" + std::to_string(workspace_bytes) +
                                                          " < " +
                                                          std::to_string(gdsllm_moe_gather_workspace_size(top_k, F)) +
                                                          ")");
    const size_t budget = static_cast<size_t>(max_lds_bytes());
    const size_t lds1 = static_cast<size_t>(H / 32) * kRec, lds2 = static_cast<size_t>(top_k) * (F / 32) * kRec;
    if (lds1 > budget || lds2 > budget)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": hidden or top_k*ffn too large for LDS staging");
    hipStream_t s = as_stream(stream);
    auto* gu = static_cast<uint16_t*>(workspace);
    GateUpRows rows{*gate, *up, idx, gu, static_cast<int>(F), static_cast<int>(2 * top_k * F)};
    const auto* xp = static_cast<const uint16_t*>(x);
    // Phase 1 writes every gate/up row (0 for an expert index out of range,
    // which phase 2 then skips), so the workspace needs no clearing.
    if (int rc = dispatch_lr<1>(rows, xp, static_cast<int>(H), static_cast<int>(gate->group_size), H, s)) return rc;
    const int lr = lanes_per_row(static_cast<int>(F / 32));
    const void* fn;
    switch (lr) {
        case 64: fn = reinterpret_cast<const void*>(&moe_down<64>); break;
        case 32: fn = reinterpret_cast<const void*>(&moe_down<32>); break;
        case 16: fn = reinterpret_cast<const void*>(&moe_down<16>); break;
        default: fn = reinterpret_cast<const void*>(&moe_down<8>); break;
    }
    if (int rc = prepare(fn, lds2)) return rc;
    const int passes = static_cast<int>((H + 64 / lr - 1) / (64 / lr));
    const int need = (passes + kWaves - 1) / kWaves;
    const int cap = blocks_per_cu(fn, lds2) * cu_count();
    const int grid = need < cap ? need : cap;
    auto* yp = static_cast<uint16_t*>(y);
    const auto* wp = static_cast<const uint16_t*>(routing_weights);
    const int tk = static_cast<int>(top_k);
    switch (lr) {
        case 64: hipLaunchKernelGGL(moe_down<64>, dim3(grid), dim3(kThreads), lds2, s, *down, idx, wp, gu, tk, yp); break;
        case 32: hipLaunchKernelGGL(moe_down<32>, dim3(grid), dim3(kThreads), lds2, s, *down, idx, wp, gu, tk, yp); break;
        case 16: hipLaunchKernelGGL(moe_down<16>, dim3(grid), dim3(kThreads), lds2, s, *down, idx, wp, gu, tk, yp); break;
        default: hipLaunchKernelGGL(moe_down<8>, dim3(grid), dim3(kThreads), lds2, s, *down, idx, wp, gu, tk, yp); break;
    }
    if (int rc = check_hip(hipGetLastError(), "moe_down launch")) return rc;
    return ok();
}
