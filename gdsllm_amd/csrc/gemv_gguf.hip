// Fused GGUF Q4_0 / Q8_0 dequant + GEMV for decode (batch 1..8) on gfx950.
//
// Computes what kernel_fused_q4_0_gemv / kernel_fused_q8_0_gemv compute
// (runtime/fused_gemv.cu:27-105, 142-205): y[r] = fp16(sum_k d_b*(q-8)*x[k]),
// fp32 accumulation, one fp16 rounding at the end.
//
// Design (HBM-bound: 0.5625 / 1.0625 bytes per weight):
//  * Super-block = 8 consecutive blocks of one row: 144 B (Q4_0) / 272 B (Q8_0),
//    i.e. exactly 9 / 17 16-byte chunks.  With in_dim % 256 == 0 every row is a
//    whole number of super-blocks and starts 16-byte aligned, so the weight
//    matrix is one long, aligned stream of super-blocks.
//  * A wavefront works on stages of 4 rows x 16 super-blocks.  It fetches a stage
//    with fully coalesced 16-byte loads (lane l takes chunk 64j+l), one stage
//    ahead in registers, and transposes it through a private LDS slot so each
//    lane then owns one whole super-block (lane = 16*row + column).  The 144 B /
//    272 B super-block stride is 4*odd dwords, so those ds_read_b128 are
//    bank-conflict free.
//  * Nibbles are turned into fp16 with the exponent trick: (q | 0x6400) is
//    1024+q and (q<<4 | 0x5400) is 64+q, so a packed pair costs one v_and_or
//    and feeds v_dot2_f32_f16 directly.  The activation vector is staged once
//    per workgroup in LDS, pre-permuted into exactly the pair order the
//    unpacked weights come out in, together with each block's correction
//    1032*sum(x_lo)+72*sum(x_hi) (Q4_0) or 1152*sum(x) (Q8_0), so a block
//    reduces to d * (S - c) with S the dot2 sum.
//  * The 16 partial sums of a row are reduced with cross-lane shuffles inside
//    the 16-lane DPP row; lane 0 of the row writes the fp16 result.

#include <mutex>
#include <utility>
#include <vector>

#include "common.h"

namespace gdsllm {
namespace {

enum class Fmt { Q4_0, Q8_0 };

template <Fmt F> struct Layout;
template <> struct Layout<Fmt::Q4_0> {
    static constexpr int kBlockBytes = 18;
    static constexpr int kSbBytes = 144;  // 8 blocks
    static constexpr int kSbChunks = 9;   // 16-byte chunks per super-block
};
template <> struct Layout<Fmt::Q8_0> {
    static constexpr int kBlockBytes = 34;
    static constexpr int kSbBytes = 272;
    static constexpr int kSbChunks = 17;
};

constexpr int kWaves = 4;          // wavefronts per workgroup
constexpr int kRowsPerStage = 4;   // 64 lanes = 4 rows x 16 columns
constexpr int kSbPerWindow = 16;   // super-blocks per row in one stage
// Prepared-x record per (batch, super-block): 128 packed fp16 pairs, 8 fp32
// block corrections, 16 bytes of padding.  560 B = 4*35 dwords keeps lanes
// reading consecutive records on distinct banks.
constexpr int kXRec = 560;

template <Fmt F>
constexpr int stage_bytes() { return kRowsPerStage * kSbPerWindow * Layout<F>::kSbBytes; }

template <Fmt F>
size_t lds_bytes(int nb, int s) { return static_cast<size_t>(nb) * s * kXRec + kWaves * stage_bytes<F>(); }

// 4 consecutive fp16 of x as two packed dwords (lo = elements 0,1).
__device__ __forceinline__ uint2 load4h(const uint16_t* p, bool aligned8) {
    if (aligned8) return *reinterpret_cast<const uint2*>(p);
    return make_uint2(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 16),
                      static_cast<uint32_t>(p[2]) | (static_cast<uint32_t>(p[3]) << 16));
}
__device__ __forceinline__ float lo_f(uint32_t v) { return h2f(v & 0xFFFFu); }
__device__ __forceinline__ float hi_f(uint32_t v) { return h2f(v >> 16); }

// Builds the prepared-x records for all `NB` batch rows of this call.
// Thread item = (batch b, block blk, quarter dd); four consecutive items make a
// block, so the corrections reduce over 4 adjacent lanes.
template <Fmt F, int NB>
__device__ void build_xprep(uint8_t* xprep, const uint16_t* __restrict__ X, int S, int64_t ldx, bool x_al8) {
    const int nblk = S * 8;
    const int items = NB * nblk * 4;
    for (int base = 0; base < items; base += kWaves * 64) {
        const int it = base + threadIdx.x;
        const bool live = it < items;
        const int dd = it & 3;
        const int blk = (it >> 2) % nblk;
        const int b = (it >> 2) / nblk;
        float part = 0.f;
        uint4 rec = make_uint4(0, 0, 0, 0);
        if (live) {
            const uint16_t* xb = X + b * ldx + blk * 32;
            if constexpr (F == Fmt::Q4_0) {
                // qs dword dd covers weights 4dd..4dd+3 (low nibbles) and
                // 16+4dd..16+4dd+3 (high nibbles).
                const uint2 lo = load4h(xb + 4 * dd, x_al8);
                const uint2 hi = load4h(xb + 16 + 4 * dd, x_al8);
                // pair order: (lo0,lo2) (hi0,hi2) (lo1,lo3) (hi1,hi3)
                rec.x = (lo.x & 0xFFFFu) | (lo.y << 16);
                rec.y = (hi.x & 0xFFFFu) | (hi.y << 16);
                rec.z = (lo.x >> 16) | (lo.y & 0xFFFF0000u);
                rec.w = (hi.x >> 16) | (hi.y & 0xFFFF0000u);
                part = 1032.f * (lo_f(lo.x) + hi_f(lo.x) + lo_f(lo.y) + hi_f(lo.y)) +
                       72.f * (lo_f(hi.x) + hi_f(hi.x) + lo_f(hi.y) + hi_f(hi.y));
            } else {
                // quarter dd covers qs dwords 2dd and 2dd+1 = weights 8dd..8dd+7
                const uint2 a = load4h(xb + 8 * dd, x_al8);
                const uint2 c = load4h(xb + 8 * dd + 4, x_al8);
                rec.x = (a.x & 0xFFFFu) | (a.y << 16);
                rec.y = (a.x >> 16) | (a.y & 0xFFFF0000u);
                rec.z = (c.x & 0xFFFFu) | (c.y << 16);
                rec.w = (c.x >> 16) | (c.y & 0xFFFF0000u);
                part = 1152.f * (lo_f(a.x) + hi_f(a.x) + lo_f(a.y) + hi_f(a.y) + lo_f(c.x) + hi_f(c.x) +
                                 lo_f(c.y) + hi_f(c.y));
            }
        }
        part += __shfl_xor(part, 1, 4);
        part += __shfl_xor(part, 2, 4);
        if (live) {
            const int s = blk >> 3, i = blk & 7;
            uint8_t* r = xprep + (b * S + s) * kXRec;
            *reinterpret_cast<uint4*>(r + (16 * i + 4 * dd) * 4) = rec;
            if (dd == 0) *reinterpret_cast<float*>(r + 512 + 4 * i) = part;
        }
    }
}

// Geometry of one stage: rows [r0, r0+nrows), super-blocks [sb0, sb0+nsb).
struct Stage {
    int r0, nrows, sb0, nsb, seg_chunks, magic;
};

template <Fmt F>
__device__ __forceinline__ Stage make_stage(int rg, int win, int M, int S) {
    Stage st;
    st.r0 = rg * kRowsPerStage;
    st.nrows = min(kRowsPerStage, M - st.r0);
    st.sb0 = win * kSbPerWindow;
    st.nsb = min(kSbPerWindow, S - st.sb0);
    st.seg_chunks = st.nsb * Layout<F>::kSbChunks;
    // floor(c / seg_chunks) == (c * magic) >> 20 for every chunk index
    // c < 64*17 and seg_chunks <= 272: the error c/2^20 < 1/272.
    st.magic = (1 << 20) / st.seg_chunks + 1;
    return st;
}

template <Fmt F>
__device__ __forceinline__ void load_stage(uint4 (&pre)[Layout<F>::kSbChunks], const uint8_t* __restrict__ W,
                                           int64_t row_bytes, const Stage& st, int lane) {
    const int total = st.nrows * st.seg_chunks;
    const uint8_t* base = W + static_cast<int64_t>(st.r0) * row_bytes + st.sb0 * Layout<F>::kSbBytes;
#pragma unroll
    for (int j = 0; j < Layout<F>::kSbChunks; ++j) {
        const int c = 64 * j + lane;
        if (c < total) {
            const int rl = (c * st.magic) >> 20;
            const int off = c - rl * st.seg_chunks;
            pre[j] = load_nt16(base + rl * row_bytes + off * 16);
        }
    }
}

template <Fmt F>
__device__ __forceinline__ void store_stage(const uint4 (&pre)[Layout<F>::kSbChunks], uint8_t* stage,
                                            const Stage& st, int lane) {
    const int total = st.nrows * st.seg_chunks;
#pragma unroll
    for (int j = 0; j < Layout<F>::kSbChunks; ++j) {
        const int c = 64 * j + lane;
        if (c < total) {
            const int rl = (c * st.magic) >> 20;
            const int off = c - rl * st.seg_chunks;
            *reinterpret_cast<uint4*>(stage + rl * (kSbPerWindow * Layout<F>::kSbBytes) + off * 16) = pre[j];
        }
    }
}

// Dot product of one super-block (already in registers as dwords D) with the
// prepared x records of all NB batch rows; accumulates into acc[b].
template <Fmt F, int NB>
__device__ __forceinline__ void superblock_dot(const uint32_t* D, const uint8_t* xrec0, int rec_stride,
                                               float (&acc)[NB]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t dbits;
        float Sd[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) Sd[b] = 0.f;
        if constexpr (F == Fmt::Q4_0) {
            // block i occupies bytes [18i, 18i+18) of the super-block
            uint32_t q[4];
            if (i % 2 == 0) {
                const int a = 9 * i / 2;
                dbits = D[a] & 0xFFFFu;
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) q[dd] = align2(D[a + dd], D[a + dd + 1]);
            } else {
                dbits = D[(9 * i - 1) / 2] >> 16;
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) q[dd] = D[(9 * i + 1) / 2 + dd];
            }
#pragma unroll
            for (int dd = 0; dd < 4; ++dd) {
                const uint32_t v = q[dd];
                const uint32_t vs = v >> 8;
                const uint32_t p0 = nib_lo_pair(v), p1 = nib_hi_pair(v);
                const uint32_t p2 = nib_lo_pair(vs), p3 = nib_hi_pair(vs);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const uint4 xv = *reinterpret_cast<const uint4*>(xrec0 + b * rec_stride + (16 * i + 4 * dd) * 4);
                    Sd[b] = dot2(p0, xv.x, Sd[b]);
                    Sd[b] = dot2(p1, xv.y, Sd[b]);
                    Sd[b] = dot2(p2, xv.z, Sd[b]);
                    Sd[b] = dot2(p3, xv.w, Sd[b]);
                }
            }
        } else {
            // block i occupies bytes [34i, 34i+34)
            uint32_t q[8];
            if (i % 2 == 0) {
                const int a = 17 * i / 2;
                dbits = D[a] & 0xFFFFu;
#pragma unroll
                for (int dd = 0; dd < 8; ++dd) q[dd] = align2(D[a + dd], D[a + dd + 1]);
            } else {
                dbits = D[(17 * i - 1) / 2] >> 16;
#pragma unroll
                for (int dd = 0; dd < 8; ++dd) q[dd] = D[(17 * i + 1) / 2 + dd];
            }
#pragma unroll
            for (int dd = 0; dd < 8; dd += 2) {
                // int8 -> biased byte u = q+128, then (u | 0x6400) = 1152 + q
                const uint32_t u0 = q[dd] ^ 0x80808080u, u1 = q[dd + 1] ^ 0x80808080u;
                const uint32_t p0 = (u0 & 0x00FF00FFu) | 0x64006400u;
                const uint32_t p1 = ((u0 >> 8) & 0x00FF00FFu) | 0x64006400u;
                const uint32_t p2 = (u1 & 0x00FF00FFu) | 0x64006400u;
                const uint32_t p3 = ((u1 >> 8) & 0x00FF00FFu) | 0x64006400u;
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const uint4 xv = *reinterpret_cast<const uint4*>(xrec0 + b * rec_stride + (16 * i + 2 * dd) * 4);
                    Sd[b] = dot2(p0, xv.x, Sd[b]);
                    Sd[b] = dot2(p1, xv.y, Sd[b]);
                    Sd[b] = dot2(p2, xv.z, Sd[b]);
                    Sd[b] = dot2(p3, xv.w, Sd[b]);
                }
            }
        }
        const float d = h2f(dbits);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float corr = *reinterpret_cast<const float*>(xrec0 + b * rec_stride + 512 + 4 * i);
            acc[b] = __builtin_fmaf(d, Sd[b] - corr, acc[b]);
        }
    }
}

template <Fmt F, int NB>
__global__ __launch_bounds__(kWaves * 64) void gguf_gemv_staged(const uint8_t* __restrict__ W,
                                                                 const uint16_t* __restrict__ X,
                                                                 uint16_t* __restrict__ Y, int M, int K,
                                                                 int64_t ldx, int64_t ldy, int x_al8) {
    using L = Layout<F>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int S = K >> 8;
    const int64_t row_bytes = static_cast<int64_t>(S) * L::kSbBytes;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    uint8_t* stage = smem + NB * S * kXRec + wave * stage_bytes<F>();
    const int RG = (M + kRowsPerStage - 1) / kRowsPerStage;
    const int NW = (S + kSbPerWindow - 1) / kSbPerWindow;
    const int total_waves = gridDim.x * kWaves;
    const int gw = blockIdx.x * kWaves + wave;
    const int my_rgs = gw < RG ? (RG - 1 - gw) / total_waves + 1 : 0;
    const int T = my_rgs * NW;

    const int r = lane >> 4, g = lane & 15;
    uint4 pre[L::kSbChunks];
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;

    // The first stage's weights are requested before x is staged, so the HBM
    // latency of the weights overlaps the x loads and the barrier.
    if (T > 0) load_stage<F>(pre, W, row_bytes, make_stage<F>(gw, 0, M, S), lane);
    build_xprep<F, NB>(smem, X, S, ldx, x_al8 != 0);
    __syncthreads();

    for (int t = 0; t < T; ++t) {
        const int rg = gw + (t / NW) * total_waves;
        const int win = t % NW;
        const Stage st = make_stage<F>(rg, win, M, S);
        store_stage<F>(pre, stage, st, lane);
        wave_lds_sync();
        if (t + 1 < T) {
            const int t1 = t + 1;
            load_stage<F>(pre, W, row_bytes, make_stage<F>(gw + (t1 / NW) * total_waves, t1 % NW, M, S), lane);
        }
        if (r < st.nrows && g < st.nsb) {
            uint32_t D[4 * L::kSbChunks];
            const uint8_t* sb = stage + r * (kSbPerWindow * L::kSbBytes) + g * L::kSbBytes;
#pragma unroll
            for (int j = 0; j < L::kSbChunks; ++j) {
                const uint4 v = *reinterpret_cast<const uint4*>(sb + 16 * j);
                D[4 * j] = v.x;
                D[4 * j + 1] = v.y;
                D[4 * j + 2] = v.z;
                D[4 * j + 3] = v.w;
            }
            superblock_dot<F, NB>(D, smem + (st.sb0 + g) * kXRec, S * kXRec, acc);
        }
        if (win == NW - 1) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float v = row16_sum(acc[b]);
                if (g == 0 && r < st.nrows) Y[b * ldy + st.r0 + r] = f2h_bits(v);
                acc[b] = 0.f;
            }
        }
    }
}

// Any in_dim % 32 == 0 and any alignment: one wave per row, one lane per block,
// byte loads, the reference's per-element order of operations.
template <Fmt F>
__global__ __launch_bounds__(256) void gguf_gemv_generic(const uint8_t* __restrict__ W,
                                                         const uint16_t* __restrict__ X,
                                                         uint16_t* __restrict__ Y, int M, int K, int NB,
                                                         int64_t ldx, int64_t ldy) {
    using L = Layout<F>;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int nblk = K / 32;
    const uint8_t* wr = W + static_cast<int64_t>(row) * nblk * L::kBlockBytes;
    for (int b = 0; b < NB; ++b) {
        const uint16_t* x = X + b * ldx;
        float acc = 0.f;
        for (int blk = lane; blk < nblk; blk += 64) {
            const uint8_t* p = wr + static_cast<int64_t>(blk) * L::kBlockBytes;
            const float d = h2f(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
            const uint16_t* xb = x + blk * 32;
            if constexpr (F == Fmt::Q4_0) {
                for (int j = 0; j < 16; ++j) {
                    const int byte = p[2 + j];
                    acc = __builtin_fmaf(d * static_cast<float>((byte & 15) - 8), h2f(xb[j]), acc);
                    acc = __builtin_fmaf(d * static_cast<float>((byte >> 4) - 8), h2f(xb[j + 16]), acc);
                }
            } else {
                for (int j = 0; j < 32; ++j)
                    acc = __builtin_fmaf(d * static_cast<float>(static_cast<int8_t>(p[2 + j])), h2f(xb[j]), acc);
            }
        }
        acc = group_sum<64>(acc);
        if (lane == 0) Y[b * ldy + row] = f2h_bits(acc);
    }
}

// Occupancy of a kernel instantiation at a given dynamic LDS size (cached).
int blocks_per_cu(const void* fn, size_t lds) {
    static std::mutex mu;
    static std::vector<std::pair<std::pair<const void*, size_t>, int>> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (auto& e : cache)
        if (e.first.first == fn && e.first.second == lds) return e.second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kWaves * 64, lds) != hipSuccess || n <= 0) n = 1;
    cache.push_back({{fn, lds}, n});
    return n;
}

template <Fmt F, int NB>
int launch_staged(const void* w, const uint16_t* x, uint16_t* y, int M, int K, int64_t ldx, int64_t ldy,
                  hipStream_t stream) {
    const int S = K >> 8;
    const size_t lds = lds_bytes<F>(NB, S);
    const void* fn = reinterpret_cast<const void*>(&gguf_gemv_staged<F, NB>);
    if (lds > 65536) {
        if (int rc = check_hip(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   static_cast<int>(lds)),
                               "hipFuncSetAttribute"))
            return rc;
    }
    const int RG = (M + kRowsPerStage - 1) / kRowsPerStage;
    const int need = (RG + kWaves - 1) / kWaves;
    const int cap = blocks_per_cu(fn, lds) * cu_count();
    const int grid = need < cap ? need : cap;
    const bool x_al8 = (reinterpret_cast<uintptr_t>(x) % 8 == 0) && (ldx % 4 == 0);
    hipLaunchKernelGGL((gguf_gemv_staged<F, NB>), dim3(grid), dim3(kWaves * 64), lds, stream,
                       static_cast<const uint8_t*>(w), x, y, M, K, ldx, ldy, x_al8 ? 1 : 0);
    return check_hip(hipGetLastError(), "gguf_gemv launch");
}

template <Fmt F>
int gemv(const char* name, const void* w, const void* x, void* y, int64_t out_dim, int64_t in_dim,
         int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    const std::string n(name);
    if (out_dim < 0 || in_dim < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (in_dim % 32 != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         n + ": in_dim must be a multiple of 32, got " + std::to_string(in_dim));
    if (batch < 1 || batch > 8)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": batch must be in [1, 8], got " + std::to_string(batch));
    if (out_dim == 0 || in_dim == 0) return ok();  // silent no-op, as the reference launchers
    if (!w || !x || !y) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (out_dim > (int64_t(1) << 30) || in_dim > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    if (batch > 1 && (ldx < in_dim || ldy < out_dim))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than the row length");
    if (reinterpret_cast<uintptr_t>(x) % 2 || reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": x and y must be 2-byte aligned");
    hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(out_dim), K = static_cast<int>(in_dim);
    const auto* xp = static_cast<const uint16_t*>(x);
    auto* yp = static_cast<uint16_t*>(y);
    const bool fast = (K % 256 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    int rc = GDSLLM_OK;
    if (fast) {
        const int S = K >> 8;
        const size_t budget = static_cast<size_t>(max_lds_bytes());
        int64_t b0 = 0;
        while (b0 < batch && rc == GDSLLM_OK) {
            // widest batch chunk whose prepared x fits next to the stage slots
            int nb = 8;
            while (nb > 1 && (nb > batch - b0 || lds_bytes<F>(nb, S) > budget)) nb >>= 1;
            if (lds_bytes<F>(1, S) > budget) { rc = -1; break; }
            const uint16_t* xb = xp + b0 * ldx;
            uint16_t* yb = yp + b0 * ldy;
            switch (nb) {
                case 8: rc = launch_staged<F, 8>(w, xb, yb, M, K, ldx, ldy, s); break;
                case 4: rc = launch_staged<F, 4>(w, xb, yb, M, K, ldx, ldy, s); break;
                case 2: rc = launch_staged<F, 2>(w, xb, yb, M, K, ldx, ldy, s); break;
                default: rc = launch_staged<F, 1>(w, xb, yb, M, K, ldx, ldy, s); break;
            }
            b0 += nb;
        }
        if (rc == GDSLLM_OK) return ok();
        if (rc != -1) return rc;
    }
    hipLaunchKernelGGL(gguf_gemv_generic<F>, dim3((M + 3) / 4), dim3(256), 0, s, static_cast<const uint8_t*>(w),
                       xp, yp, M, K, static_cast<int>(batch), ldx, ldy);
    if (int e = check_hip(hipGetLastError(), (n + " launch").c_str())) return e;
    return ok();
}

}  // namespace
}  // namespace gdsllm

using namespace gdsllm;

extern "C" int gdsllm_fused_q4_0_gemv(const void* weight, const void* x, void* y, int64_t out_dim,
                                      int64_t in_dim, int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    return gemv<Fmt::Q4_0>("fused_q4_0_gemv", weight, x, y, out_dim, in_dim, batch, ldx, ldy, stream);
}

extern "C" int gdsllm_fused_q8_0_gemv(const void* weight, const void* x, void* y, int64_t out_dim,
                                      int64_t in_dim, int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    return gemv<Fmt::Q8_0>("fused_q8_0_gemv", weight, x, y, out_dim, in_dim, batch, ldx, ldy, stream);
}
