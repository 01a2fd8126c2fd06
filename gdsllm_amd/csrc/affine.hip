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

#include <type_traits>

#include <mutex>

#include "common.h"
#include "topk.h"

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
// Returns whether this thread met an x that is not finite.
template <int NB>
__device__ bool build_xprep_plain(uint8_t* xp, const uint16_t* __restrict__ X, int chunks, int64_t ldx, bool al16) {
    const int items = NB * chunks * 4;
    bool nonfinite = false;
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
        nonfinite |= live && !__builtin_isfinite(sum);
    }
    return nonfinite;
}

// Exact nibbles: the unpacked pairs (1024 + q, 64 + q) enter the dot
// products as q itself (one packed fp16 subtract per pair, exact), so the fp32
// sum runs over nib * x with the reference's magnitudes; the chunk is then
// s * sum(nib * x) + b * sum(x) and the offset correction drops out.  The
// offset form sum((1024 + q) * x) - 1024 * sum(x) loses about 10 bits to
// cancellation when one x dwarfs the rest (an activation near 65504).  A row
// whose sum is not finite (an infinite or NaN x, where the factored form and
// the reference's per-element (nib*s + b)*x differ) is recomputed by
// affine_row_exact.
constexpr bool kAffineExact = true;
constexpr uint32_t kNeg1024 = 0xE400E400u;  // fp16 -1024 in both halves
constexpr uint32_t kNeg64 = 0xD400D400u;    // -64
__device__ __forceinline__ uint32_t unbias_nib(uint32_t a, uint32_t neg_bias_pair) {
    if constexpr (!kAffineExact) return a;
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, a) + __builtin_bit_cast(half2_t, neg_bias_pair));
}

// Dot of one 32-element chunk with its prepared record: s*(S - corr) + b*sum
// (s*S + b*sum with exact nibbles).
__device__ __forceinline__ float chunk_dot(uint4 w, const uint8_t* rec, float s, float b) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    float S = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 xv = *reinterpret_cast<const uint4*>(rec + 16 * q);
        const uint32_t v = wd[q], vs = v >> 8;
        S = dot2(unbias_nib(nib_lo_pair(v), kNeg1024), xv.x, S);
        S = dot2(unbias_nib(nib_hi_pair(v), kNeg64), xv.y, S);
        S = dot2(unbias_nib(nib_lo_pair(vs), kNeg1024), xv.z, S);
        S = dot2(unbias_nib(nib_hi_pair(vs), kNeg64), xv.w, S);
    }
    const float2 cs = *reinterpret_cast<const float2*>(rec + 64);
    return __builtin_fmaf(s, kAffineExact ? S : S - cs.x, b * cs.y);
}

// The reference's per-element arithmetic for one row (kernel_fused_affine_q4_gemv,
// runtime/affine_q4_dequant.cu:118-128): sum over k of (nib*s + b)*x[k] in
// fp32, one lane, serially.  The slow path for a row whose fast sum is not
// finite, so that +-inf and NaN come out where the reference's do.
__device__ __forceinline__ float affine_row_exact(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                               const uint16_t* __restrict__ b, const uint16_t* __restrict__ x, int K,
                                               int gsize) {
    float acc = 0.f;
    for (int i = 0; i < K / 8; ++i) {
        const uint32_t v = w[i];
        const int G = (8 * i) / gsize;
        const float sf = h2f(s[G]), bf = h2f(b[G]);
        for (int n = 0; n < 8; ++n) {
            const float val = fp32_rounded(static_cast<float>((v >> (4 * n)) & 15u) * sf + bf);
            acc = __builtin_fmaf(val, h2f(x[8 * i + n]), acc);
        }
    }
    return acc;
}

// Where one row of a GEMV lives and where its result goes.
struct PlainRows {
    const uint32_t* W;
    const uint16_t* S;
    const uint16_t* B;
    uint16_t* Y;
    int64_t ldy;
    int M;
    __device__ int lane_index(int) const { return 0; }
    __device__ bool locate(int row, const uint32_t*& w, const uint16_t*& s, const uint16_t*& b, int K, int gpr,
                           int = 0) const {
        w = W + static_cast<int64_t>(row) * (K / 8);
        s = S + static_cast<int64_t>(row) * gpr;
        b = B + static_cast<int64_t>(row) * gpr;
        return true;
    }
    __device__ void store(int bidx, int row, float v) const { Y[bidx * ldy + row] = f2h_bits(v); }
    __device__ bool locate_lane(int row, const uint32_t*& w, const uint16_t*& s, const uint16_t*& b, int K,
                                int gpr) const {
        return locate(row, w, s, b, K, gpr);
    }
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
    __device__ bool locate_lane(int row, const uint32_t*& w, const uint16_t*& s, const uint16_t*& b, int K,
                                int gpr) const {
        return locate(row, w, s, b, K, gpr);
    }
};

// Dynamic LDS a kernel of this file may take: the device's limit less what
// the workgroup-wide flag reduction (__syncthreads_or) keeps for itself.
inline size_t lds_budget() { return static_cast<size_t>(max_lds_bytes()) - 256; }

// Rows whose x (or h) holds an infinite or NaN value take the reference's
// per-element arithmetic instead of the factored s*sum(nib*x) + b*sum(x):
// nib = 0 gives 0*inf = NaN in the factored form where the reference has
// b*inf.  The whole workgroup (or wave) switches when any element of its x is
// not finite, in a branch of its own, so the fast loop keeps its registers.

// Row `row` of `rows`, batch row bidx of x, per element (one lane).
template <class Rows>
__device__ __forceinline__ void store_exact_row(const Rows& rows, int bidx, int row, const uint16_t* __restrict__ X,
                                                int64_t ldx, int K, int gsize) {
    const uint32_t* w;
    const uint16_t *s, *b;
    const float v = rows.locate_lane(row, w, s, b, K, K / gsize) ? affine_row_exact(w, s, b, X + bidx * ldx, K, gsize)
                                                                 : 0.f;
    rows.store(bidx, row, v);
}

// One output row o of the gather's phase 2 with the reference's per-element
// arithmetic: sum over the valid slots k of w_k * (down[e_k][o] . h_k).  Slots
// k < top_k take expert idx[k] and weight rw[k]; with `shared` the one slot is
// expert 0 of `down` (the shared expert's descriptors) with weight 1 and h
// slot top_k.  h_k: with FROM_GU the fp16 gate/up outputs [k][2][F] at src
// (h = fp16(fp16(silu(g)) * u)), else h [k][F] at src.  The slow path for a
// row whose fast sum is not finite.
template <bool FROM_GU>
__device__ __forceinline__ float moe_down_row_exact(const gdsllm_affine_experts& down,
                                                    const int32_t* __restrict__ idx,
                                                    const uint16_t* __restrict__ rw, int top_k, int o,
                                                    const uint16_t* __restrict__ src, bool shared) {
    const int F = static_cast<int>(down.in_dim), gsize = static_cast<int>(down.group_size), gpr = F / gsize;
    float acc = 0.f;
    const int nk = shared ? 1 : top_k;
    for (int k = 0; k < nk; ++k) {
        const int e = shared ? 0 : idx[k];
        if (e < 0 || e >= down.num_experts) continue;
        const int hk = shared ? top_k : k;
        const uint32_t* w = reinterpret_cast<const uint32_t*>(static_cast<const char*>(down.weight) +
                                                              e * down.weight_stride) + static_cast<int64_t>(o) * (F / 8);
        const uint16_t* sp = reinterpret_cast<const uint16_t*>(static_cast<const char*>(down.scales) +
                                                               e * down.scale_stride) + static_cast<int64_t>(o) * gpr;
        const uint16_t* bp = reinterpret_cast<const uint16_t*>(static_cast<const char*>(down.biases) +
                                                               e * down.bias_stride) + static_cast<int64_t>(o) * gpr;
        float dot = 0.f;
        for (int i = 0; i < F / 8; ++i) {
            const uint32_t v = w[i];
            const int G = (8 * i) / gsize;
            const float sf = h2f(sp[G]), bf = h2f(bp[G]);
            for (int n = 0; n < 8; ++n) {
                const int jj = 8 * i + n;
                float h;
                if constexpr (FROM_GU) {
                    const float g = h2f(src[static_cast<int64_t>(hk) * 2 * F + jj]);
                    const float sg = h2f(f2h_bits(g / (1.0f + expf(-g))));
                    h = h2f(f2h_bits(sg * h2f(src[static_cast<int64_t>(hk) * 2 * F + F + jj])));
                } else {
                    h = h2f(src[static_cast<int64_t>(hk) * F + jj]);
                }
                dot = __builtin_fmaf(fp32_rounded(static_cast<float>((v >> (4 * n)) & 15u) * sf + bf), h, dot);
            }
        }
        acc = __builtin_fmaf(shared ? 1.0f : h2f(rw[k]), dot, acc);
    }
    return acc;
}

// Generic affine GEMV: LR lanes share a row (64/LR rows per wave pass), each
// lane walks chunks lane%LR, +LR, ... of its row; loads are issued kU items
// ahead of the math.  NB batch rows of x share every weight load.
template <int LR, int NB, class Rows>
__global__ __launch_bounds__(kThreads) void affine_gemv(Rows rows, const uint16_t* __restrict__ X, int K, int gsize,
                                                        int64_t ldx, int x_al16) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int CPR = K / 32;
    const bool nonfinite = __syncthreads_or(build_xprep_plain<NB>(smem, X, CPR, ldx, x_al16 != 0));

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
    if (nonfinite) {
        // lane l < RW takes row l of each of this wave's passes
        for (int pass = gw; pass < passes; pass += TW) {
            const int row = pass * RW + lane;
            if (lane < RW && row < rows.M)
                for (int b = 0; b < NB; ++b) store_exact_row(rows, b, row, X, ldx, K, gsize);
        }
        return;
    }

    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;

    for (int base = 0; base < n_items; base += kU) {
        uint4 wv[kU];
        uint32_t sv[kU], bv[kU];
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
                    sv[u] = s[G];  // raw bits, converted at use (no early wait)
                    bv[u] = b[G];
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
                    acc[b] += chunk_dot(wv[u], smem + (b * CPR + c) * kRec, h2f(sv[u]), h2f(bv[u]));
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
    bool h_nonfinite = false;
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
            h_nonfinite |= live && !__builtin_isfinite(sum);
        }
    }
    const bool nonfinite = __syncthreads_or(h_nonfinite);

    constexpr int RW = 64 / LR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LR, li = lane % LR;
    const int gpr = F / gsize;
    const int CPL = (CPR + LR - 1) / LR;
    const int passes = (H + RW - 1) / RW;
    const int TW = gridDim.x * kWaves;
    const int gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (nonfinite) {
        for (int pass = gw; pass < passes; pass += TW) {
            const int o = pass * RW + lane;
            if (lane < RW && o < H) Y[o] = f2h_bits(moe_down_row_exact<true>(down, idx, rw, top_k, o, gu, false));
        }
        return;
    }
    for (int pass = gw; pass < passes; pass += TW) {
        const int o = pass * RW + sub;
        float acc = 0.f;
        for (int t = 0; t < CPL; ++t) {
            const int c = li + LR * t;
            for (int k0 = 0; k0 < top_k; k0 += kU) {
                uint4 wv[kU];
                uint32_t sv[kU], bv[kU], wk[kU];
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
                            sv[u] = s[G];  // raw bits, converted at use (no early wait)
                            bv[u] = b[G];
                            wk[u] = rw[k];
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < kU; ++u)
                    if (ok[u])
                        acc = __builtin_fmaf(h2f(wk[u]), chunk_dot(wv[u], smem + ((k0 + u) * CPR + c) * kRec, h2f(sv[u]), h2f(bv[u])),
                                             acc);
            }
        }
        acc = group_sum<LR>(acc);
        if (li == 0 && o < H) {
            Y[o] = f2h_bits(acc);
        }
    }
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
    if (int rc = prepare_lds(fn, lds)) return rc;
    const int passes = (rows.M + 64 / LR - 1) / (64 / LR);
    const int need = (passes + kWaves - 1) / kWaves;
    const int cap = blocks_per_cu(fn, lds, kThreads) * cu_count();
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


// ---- row-span kernels ------------------------------------------------------------
// Lane li of a row owns the chunks li, li+LR, ... (CPL of them) of every row it
// touches, so its prepared slice of x stays in registers for the whole kernel.
// A 16-byte affine chunk is aligned and lies inside one group, so lanes load
// their chunks directly: LR consecutive lanes cover LR consecutive chunks
// (coalesced), no LDS transpose.  A wave's stage is 4 load groups of 64/LR
// rows; the first stage is requested before x is prepared, the next one while
// the current one is computed, and the 4 partial sums of each lane reduce with
// two exchange-halving swaps and DPP steps.

constexpr uint32_t kPair1024 = 0x64006400u;  // (1024, 1024)
constexpr uint32_t kPair64 = 0x54005400u;    // (64, 64)
constexpr uint32_t kPairOne = 0x3C003C00u;   // (1, 1)

// Prepared x of one 32-element chunk in registers: pairs in chunk_dot order,
// offset correction 1024*sum(x_even) + 64*sum(x_odd) within each word, and sum(x).
struct XChunk {
    uint32_t p[16];
    float corr, sum;
};

// 32 raw fp16 of a chunk (r[i] = x[2i], x[2i+1]); zeros when not live.
__device__ __forceinline__ void load_xchunk_raw(uint32_t (&r)[16], const uint16_t* __restrict__ src, bool al16,
                                                bool live) {
    if (live && al16) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * k);
            r[4 * k] = v.x;
            r[4 * k + 1] = v.y;
            r[4 * k + 2] = v.z;
            r[4 * k + 3] = v.w;
        }
    } else if (live) {
#pragma unroll
        for (int i = 0; i < 16; ++i) r[i] = static_cast<uint32_t>(src[2 * i]) | (static_cast<uint32_t>(src[2 * i + 1]) << 16);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) r[i] = 0u;
    }
}

__device__ __forceinline__ void make_xchunk(XChunk& xc, const uint32_t (&r)[16]) {
    float corr = 0.f, sum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        // word q = elements 8q..8q+7: pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7)
        const uint32_t a = r[4 * q], b = r[4 * q + 1], c = r[4 * q + 2], d = r[4 * q + 3];
        xc.p[4 * q + 0] = __builtin_amdgcn_perm(c, a, 0x05040100u);
        xc.p[4 * q + 1] = __builtin_amdgcn_perm(c, a, 0x07060302u);
        xc.p[4 * q + 2] = __builtin_amdgcn_perm(d, b, 0x05040100u);
        xc.p[4 * q + 3] = __builtin_amdgcn_perm(d, b, 0x07060302u);
        corr = dot2(xc.p[4 * q + 0], kPair1024, corr);
        corr = dot2(xc.p[4 * q + 2], kPair1024, corr);
        corr = dot2(xc.p[4 * q + 1], kPair64, corr);
        corr = dot2(xc.p[4 * q + 3], kPair64, corr);
#pragma unroll
        for (int k = 0; k < 4; ++k) sum = dot2(xc.p[4 * q + k], kPairOne, sum);
    }
    xc.corr = corr;
    xc.sum = sum;
}

// s*(S - corr) + b*sum for one chunk w against x pairs p.
__device__ __forceinline__ float chunk_dot_p(uint4 w, const uint32_t* p, float corr, float sum, float s, float b,
                                             const NibUnpack& nu) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    float S = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t v = wd[q], vs = v >> 8;
        if constexpr (kAffineExact) {
            S = dot2(unbias_nib(nu.lo_c(v), kNeg1024), p[4 * q + 0], S);
            S = dot2(unbias_nib(nu.hi_c(v), kNeg64), p[4 * q + 1], S);
            S = dot2(unbias_nib(nu.lo_c(vs), kNeg1024), p[4 * q + 2], S);
            S = dot2(unbias_nib(nu.hi_c(vs), kNeg64), p[4 * q + 3], S);
        } else {
            S = dot2(nu.lo(v), p[4 * q + 0], S);
            S = dot2(nu.hi(v), p[4 * q + 1], S);
            S = dot2(nu.lo(vs), p[4 * q + 2], S);
            S = dot2(nu.hi(vs), p[4 * q + 3], S);
        }
    }
    return __builtin_fmaf(s, kAffineExact ? S : S - corr, b * sum);
}

// Sum over aligned groups of N lanes (N = 1, 2, 4, 8, 16), every lane of the
// group receiving the total; VALU-only DPP steps.
template <int N>
__device__ __forceinline__ float lanes_sum(float v) {
    if constexpr (N >= 2) v += dpp_read<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (N >= 4) v += dpp_read<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (N >= 8) v += dpp_read<0x141>(v);  // row_half_mirror
    if constexpr (N >= 16) v += dpp_read<0x140>(v); // row_mirror
    return v;
}

// acc[0..3] summed over the LR lanes of each aligned lane group.  Lane li
// (= lane % LR) ends up with the total of value j = 2*bit(li, LR/2) +
// bit(li, LR/4); lanes with li % (LR/4) == 0 hold one value each.
template <int LR>
__device__ __forceinline__ float reduce4(const float (&acc)[4], int lane) {
    constexpr int H1 = LR / 2, H2 = LR / 4;
    const bool b1 = lane & H1;
    float k0 = b1 ? acc[2] : acc[0], k1 = b1 ? acc[3] : acc[1];
    const float s0 = b1 ? acc[0] : acc[2], s1 = b1 ? acc[1] : acc[3];
    k0 += __shfl_xor(s0, H1);
    k1 += __shfl_xor(s1, H1);
    const bool b2 = lane & H2;
    float k = b2 ? k1 : k0;
    k += __shfl_xor(b2 ? k0 : k1, H2);
    return lanes_sum<H2>(k);
}
template <int LR>
__device__ __forceinline__ int reduce4_index(int lane) {
    return 2 * ((lane & (LR / 2)) ? 1 : 0) + ((lane & (LR / 4)) ? 1 : 0);
}

// Gate/up rows of the selected experts as one virtual matrix, gate and up of
// the same FFN row adjacent: virtual row v -> slot k = v / (2F), FFN row
// n = (v % 2F) / 2, projection v & 1 (0 = gate, 1 = up).  Outputs: g/u fp16
// [top_k][2][F], and h = fp16(fp16(silu(g)) * u) fp16 [top_k][F].
// The shared expert of the fused decode step (one-expert descriptors) fills
// slot shared_slot, after the routed slots.
// With router logits (routed step), every wave takes the top-k itself from
// the fp16 logits of all route_e experts (top_k = shared_slot picks, the
// selection of route_topk, topk.h), and the grid's first wave also stores
// the picks and their fp16 softmax weights for the down launch and the
// caller.
struct SharedSlot {
    gdsllm_affine_experts sgate, sup;
    int shared_slot;
    const uint16_t* gate_w;  // fp16 [K] shared-expert gate row
    uint16_t* logit;         // fp16 out: its logit on x
    const uint16_t* route_logits;  // fp16 [route_e], or null: picks come from idx
    int route_e;                   // experts routed over (<= kRouteMaxExperts, multiple of 8)
    int32_t* route_idx;            // out: the top_k picks, descending
    uint16_t* route_w;             // out: their fp16 softmax weights
};
constexpr int kRouteMaxExperts = 512;  // 8 logits per lane
struct NoSharedSlot {};

template <bool SH>
struct GateUpPairsT : std::conditional_t<SH, SharedSlot, NoSharedSlot> {
    gdsllm_affine_experts gate, up;
    const int32_t* idx;
    uint16_t* gu;
    uint16_t* h;
    int F;
    int M;
    // Lane l holds idx[l] (the slot count is at most 64), read once per wave;
    // the shared slot reads expert 0 of its own descriptors.
    __device__ int lane_index(int lane) const {
        if constexpr (SH)
            if (lane == this->shared_slot) return 0;
        return lane < M / (2 * F) ? idx[lane] : -1;
    }
    // lane_index of the routed step: the wave's own top-k of the router
    // logits (lane l holds logits 8l .. 8l+7, one 16-byte load); the writer
    // wave stores the picks and weights.
    __device__ uint4 route_load(int lane) const {
        return load_nt16(this->route_logits + 8 * (8 * lane < this->route_e ? lane : 0));
    }
    __device__ int route_lane(uint4 v, int lane, bool writer) const {
        static_assert(SH, "routing is part of the fused step");
        const int E = this->route_e, k = this->shared_slot;
        const bool in = 8 * lane < E;
        const uint32_t hv[4] = {v.x, v.y, v.z, v.w};
        uint32_t word[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) word[j] = in ? pick_word((hv[j >> 1] >> (16 * (j & 1))) & 0xFFFFu, 8 * lane + j) : 0u;
        int my_idx;
        uint32_t my_key, top_key;
        topk_select<8>(word, k, lane, my_idx, my_key, top_key);
        if (writer) {
            const uint16_t w = topk_weight(my_key, top_key, k, lane);
            if (lane < k) {
                this->route_idx[lane] = my_idx;
                this->route_w[lane] = w;
            }
        }
        if (lane == this->shared_slot) return 0;
        return lane < k ? my_idx : -1;
    }
    __device__ const gdsllm_affine_experts& proj(int k, bool is_up) const {
        if constexpr (SH)
            if (k == this->shared_slot) return is_up ? this->sup : this->sgate;
        return is_up ? up : gate;
    }
    // v is the same for the whole wave (one row per load group), so the
    // expert index is a lane read, not a dependent global load.
    __device__ bool locate(int v, const uint32_t*& w, const uint16_t*& s, const uint16_t*& b, int K, int gpr,
                           int lane_idx) const {
        // v, and so the slot and projection, are wave-uniform: said outright,
        // the descriptor is chosen in scalar registers (computed per lane, the
        // shared variant read it with a vector load whose wait drained every
        // weight load in flight)
        const int vu = __builtin_amdgcn_readfirstlane(v);
        const int k = vu / (2 * F);
        const int rem = vu - k * 2 * F;
        const int n = rem >> 1;
        const gdsllm_affine_experts& p = proj(k, rem & 1);
        const int e = __builtin_amdgcn_readlane(lane_idx, k);
        if (e < 0 || e >= p.num_experts) return false;
        w = reinterpret_cast<const uint32_t*>(static_cast<const char*>(p.weight) + e * p.weight_stride) +
            static_cast<int64_t>(n) * (K / 8);
        s = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.scales) + e * p.scale_stride) +
            static_cast<int64_t>(n) * gpr;
        b = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.biases) + e * p.bias_stride) +
            static_cast<int64_t>(n) * gpr;
        return true;
    }
    __device__ void store(int, int v, float val) const {
        const int k = v / (2 * F);
        const int rem = v - k * 2 * F;
        gu[(2 * k + (rem & 1)) * F + (rem >> 1)] = f2h_bits(val);
    }
    // locate for one lane on its own, its slot's expert e given (the
    // lane_index of lane v / 2F): the slow path
    __device__ bool locate_pair_lane(int v, int e, const uint32_t*& w, const uint16_t*& s, const uint16_t*& b, int K,
                                     int gpr) const {
        const int k = v / (2 * F);
        const int rem = v - k * 2 * F;
        const int n = rem >> 1;
        const gdsllm_affine_experts& p = proj(k, rem & 1);
        if (e < 0 || e >= p.num_experts) return false;
        w = reinterpret_cast<const uint32_t*>(static_cast<const char*>(p.weight) + e * p.weight_stride) +
            static_cast<int64_t>(n) * (K / 8);
        s = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.scales) + e * p.scale_stride) +
            static_cast<int64_t>(n) * gpr;
        b = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.biases) + e * p.bias_stride) +
            static_cast<int64_t>(n) * gpr;
        return true;
    }
};
using GateUpPairs = GateUpPairsT<false>;
using GateUpPairsShared = GateUpPairsT<true>;

template <class Rows> struct IsGateUp { static constexpr bool value = false; };
template <bool SH> struct IsGateUp<GateUpPairsT<SH>> { static constexpr bool value = true; };

template <int LR, int CPL, int NB, class Rows>
__global__ __launch_bounds__(kThreads) void affine_rows(Rows rows, const uint16_t* __restrict__ X, int K, int gsize,
                                                        int64_t ldx, int x_al16) {
    constexpr int RPG = 64 / LR;  // rows per load group
    // load groups per stage: gate/up pairs take one pair (gate row n, up row
    // n) per stage, loaded after the previous stage is computed; plain rows
    // take 4 rows per stage with the next stage requested before the compute
    constexpr bool kPairs = IsGateUp<Rows>::value;
    constexpr int G = kPairs ? 2 : 4;
    constexpr int RPS = G * RPG;  // rows per stage
    static_assert(!IsGateUp<Rows>::value || (LR == 64 && NB == 1), "gate/up pairs need one row per load group");
    const int lane = threadIdx.x & 63;
    const int li = lane % LR, sub = lane / LR;
    const int CPR = K >> 5, gpr = K / gsize;
    const int stages = (rows.M + RPS - 1) / RPS;
    const int TW = gridDim.x * kWaves;
    const int gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int T = gw < stages ? (stages - 1 - gw) / TW + 1 : 0;
    constexpr bool kRoutable = std::is_same_v<Rows, GateUpPairsT<true>>;
    uint32_t xr[NB][CPL][16];
    auto load_x = [&] {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = li + LR * i;
                load_xchunk_raw(xr[b][i], X + b * ldx + 32 * c, x_al16 != 0, c < CPR);
            }
    };
    int routed_idx = -1;
    if constexpr (kRoutable) {
        // x in flight through the routing and the gate logit
        load_x();
        if (rows.route_logits) {
            // routed step: one wave of the workgroup takes the top-k (wave
            // blockIdx % 4, so the routing waves of a CU's workgroups sit on
            // different SIMDs) and hands the picks to the others through LDS;
            // every wave of the workgroup is still here for the barrier
            __shared__ int route_pick[64];
            if ((threadIdx.x >> 6) == static_cast<int>(blockIdx.x & (kWaves - 1)))
                route_pick[lane] = rows.route_lane(rows.route_load(lane), lane, blockIdx.x == 0);
            __syncthreads();
            routed_idx = route_pick[lane];
        }
        // the shared-expert gate logit, by the grid's last workgroup (its
        // waves have the fewest stages): wave j takes part j of the row dot
        // and wave 0 adds the parts in order, as gdsllm_gemv_f16 does (one
        // wave taking all four parts made itself the launch's last wave)
        if (blockIdx.x == gridDim.x - 1) {
            __shared__ float logit_part[kWaves];
            static_assert(kWaves == 4, "one part of the row dot per wave");
            const int part = threadIdx.x >> 6;
            const float p = group_sum<64>(f16_part_lane(rows.gate_w, X, K, part, lane));
            if (lane == 0) logit_part[part] = p;
            __syncthreads();
            if (threadIdx.x == 0)
                *rows.logit = f2h_bits(((logit_part[0] + logit_part[1]) + logit_part[2]) + logit_part[3]);
        }
        if (T == 0) {
            wait_vmcnt<0>();  // no load outlives its wave
            return;
        }
    } else {
        if (T == 0) return;
    }
    const NibUnpack nu;

    // Scale / bias bits stay raw until the compute: converting them here would
    // make the wave wait for every load issued before them (loads retire in
    // order), turning the prefetch into a stall.
    uint4 wv[G][CPL];
    uint32_t sv[G][CPL], bv[G][CPL];
    bool ok[G];
    // the slot experts: idx[lane], or (routed step) the workgroup's top-k
    int lane_idx = -1;
    auto issue = [&](int st) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int row = st * RPS + j * RPG + sub;
            const uint32_t* w = nullptr;
            const uint16_t *sp = nullptr, *bp = nullptr;
            ok[j] = row < rows.M && rows.locate(row, w, sp, bp, K, gpr, lane_idx);
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = li + LR * i;
                if (ok[j] && c < CPR) {
                    wv[j][i] = load_nt16(w + 4 * c);
                    const int gi = (32 * c) / gsize;
                    sv[j][i] = sp[gi];
                    bv[j][i] = bp[gi];
                }
            }
        }
    };
    // x first, then the first stage's weights: preparing x waits only for x
    if constexpr (!kRoutable) load_x();
    if constexpr (kRoutable)
        lane_idx = rows.route_logits ? routed_idx : rows.lane_index(lane);
    else
        lane_idx = rows.lane_index(lane);
    // Gate/up pairs: the expert indices (lane_idx) and x in before any weight
    // is requested.  Waiting for them here, once, lets every later read of
    // lane_idx go without a wait; otherwise the compiler, unsure how many
    // (conditional) weight loads follow it, drains all of them before each
    // load group.  It also keeps x from queueing behind the weights.
    if constexpr (kPairs) wait_vmcnt<0>();
    issue(gw);
    XChunk xc[NB][CPL];
    bool x_nonfinite = false;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            make_xchunk(xc[b][i], xr[b][i]);
            x_nonfinite |= !__builtin_isfinite(xc[b][i].sum);
        }
    if (__builtin_amdgcn_ballot_w64(x_nonfinite) != 0) {
        // the reference's per-element arithmetic for this wave's rows: lane l
        // takes row l of each stage (gate/up pairs: the even lane both rows of
        // its pair, then h)
        wait_vmcnt<0>();
        for (int t = 0; t < T; ++t) {
            const int row = (gw + t * TW) * RPS + lane;
            if constexpr (IsGateUp<Rows>::value) {
                // the slot's expert from the lane that holds it, read with every lane active
                const int e = __shfl(lane_idx, (row / (2 * rows.F)) & 63);
                if (lane < RPS && (lane & 1) == 0 && row + 1 < rows.M) {
                    const uint32_t *wg, *wu;
                    const uint16_t *sg, *bg, *su, *bu;
                    const float g = rows.locate_pair_lane(row, e, wg, sg, bg, K, gpr) ? affine_row_exact(wg, sg, bg, X, K, gsize) : 0.f;
                    const float u = rows.locate_pair_lane(row + 1, e, wu, su, bu, K, gpr) ? affine_row_exact(wu, su, bu, X, K, gsize) : 0.f;
                    rows.store(0, row, g);
                    rows.store(0, row + 1, u);
                    const int k = row / (2 * rows.F);
                    rows.h[k * rows.F + ((row - k * 2 * rows.F) >> 1)] = silu_mul_h(g, u);
                }
            } else {
                if (lane < RPS && row < rows.M)
                    for (int b = 0; b < NB; ++b) store_exact_row(rows, b, row, X, ldx, K, gsize);
            }
        }
        return;
    }

    for (int t = 0; t < T; ++t) {
        const int st = gw + t * TW;
        uint4 cw[G][CPL];
        uint32_t cs[G][CPL], cb[G][CPL];
        bool cok[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            cok[j] = ok[j];
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                cw[j][i] = wv[j][i];
                cs[j][i] = sv[j][i];
                cb[j][i] = bv[j][i];
            }
        }
        if (!kPairs && t + 1 < T) issue(st + TW);
        float acc[NB][G];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < G; ++j) acc[b][j] = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const bool cl = li + LR * i < CPR;
#pragma unroll
            for (int j = 0; j < G; ++j)
                if (cok[j] && cl) {
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        acc[b][j] += chunk_dot_p(cw[j][i], xc[b][i].p, xc[b][i].corr, xc[b][i].sum, h2f(cs[j][i]),
                                                 h2f(cb[j][i]), nu);
                }
        }
        if constexpr (kPairs) {
            // one row per half-wave (LR = 64): lanes 0-31 the gate row, 32-63 the up row
            const bool b1 = lane & 32;
            float v = b1 ? acc[0][1] : acc[0][0];
            v += __shfl_xor(b1 ? acc[0][0] : acc[0][1], 32);
            v += __shfl_xor(v, 16);
            v = lanes_sum<16>(v);
            const int row = st * RPS + (b1 ? 1 : 0);
            if ((lane & 31) == 0 && row < rows.M) rows.store(0, row, v);
            const float up = __shfl_xor(v, 32);
            if (lane == 0 && row < rows.M) {
                const int k = row / (2 * rows.F);
                const int n = (row - k * 2 * rows.F) >> 1;
                rows.h[k * rows.F + n] = silu_mul_h(v, up);
            }
            if (t + 1 < T) issue(st + TW);
        } else {
            const int j = reduce4_index<LR>(lane);
            const int row = st * RPS + j * RPG + sub;
            const bool writer = (li % (LR / 4)) == 0 && row < rows.M;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float v = reduce4<LR>(acc[b], lane);
                if (writer) rows.store(b, row, v);
            }
        }
    }
}

// Phase 2 of the gather MLP.  Lane li of a group of LR = F/32 lanes owns chunk
// li of the down-projection rows of expert slot k = i*(64/LR) + lane/LR for
// i < SLOTS, i.e. a fixed (expert, chunk) pair per slot, for every output
// row.  h of all selected experts is prepared once per workgroup in LDS
// (records as in affine_gemv).  A stage is R output rows: R*SLOTS chunk loads
// per lane, issued before h is prepared for the first stage.
//
// With a shared expert (nsh = 1: sdown, one expert, in slot top_k of h and of
// the lane slots, gl its fp16 gate logit) the lanes of that slot accumulate
// the shared down row separately, and the row's writer applies
// y = clamp(fp16(routed) + fp16(fp16(sigmoid(g)) * fp16(shared))) with the
// rounding of moe_combine (torch's fp16 elementwise ops, qwen_moe.py:508-513).
template <int LR, int SLOTS, int NT, bool SH>
__global__ __launch_bounds__(NT) void moe_down_rows(gdsllm_affine_experts down, const int32_t* __restrict__ idx,
                                                          const uint16_t* __restrict__ rw,
                                                          const uint16_t* __restrict__ hbuf, int top_k,
                                                          uint16_t* __restrict__ Y, gdsllm_affine_experts sdown,
                                                          const uint16_t* __restrict__ gl) {
    // SH: a separate instantiation, so the gather without a shared expert
    // keeps its registers (the extra accumulator made it spill)
    constexpr int nsh = SH ? 1 : 0;
    constexpr int EPI = 64 / LR;
    constexpr int R = SLOTS <= 4 ? 2 : 1;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int F = static_cast<int>(down.in_dim);
    const int H = static_cast<int>(down.out_dim);
    const int gsize = static_cast<int>(down.group_size);
    const int CPR = F >> 5, gpr = F / gsize;
    const int lane = threadIdx.x & 63;
    const int li = lane % LR, sub = lane / LR;
    constexpr int NWV = NT / 64;  // waves per workgroup
    const int stages = (H + R - 1) / R;
    const int TW = gridDim.x * NWV;
    const int gw = blockIdx.x * NWV + (threadIdx.x >> 6);
    const int T = gw < stages ? (stages - 1 - gw) / TW + 1 : 0;
    const NibUnpack nu;

    // Request order: expert indices and routing weights, then this thread's
    // first h items, then (once the indices are in) the first stage's weights;
    // loads retire in order, so each consumer waits only for what it needs.
    // Every load here is unconditional (indices clamped to valid addresses,
    // what is out of range discarded afterwards): a load under a branch leaves
    // the compiler unsure how many loads follow it, and it then waits for all
    // of them before the first use, i.e. for the weights before h is prepared.
    int eraw[SLOTS];
    uint32_t wraw[SLOTS];
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
        const int k = i * EPI + sub;
        const int kc = k < top_k ? k : 0;
        eraw[i] = idx[kc];
        wraw[i] = rw[kc];
    }
    const uint32_t graw = nsh ? gl[0] : 0u;
    constexpr int kEarly = NT >= 1024 ? 2 : 3;
    const int items = (top_k + nsh) * CPR * 4;
    uint4 hraw[kEarly];
#pragma unroll
    for (int u = 0; u < kEarly; ++u) {
        const int it0 = u * NT + threadIdx.x;
        const int it = it0 < items ? it0 : 0;
        const int wq = it & 3, c = (it >> 2) % CPR, k = (it >> 2) / CPR;
        hraw[u] = *reinterpret_cast<const uint4*>(hbuf + k * F + 32 * c + 8 * wq);
    }

    // expert slot of each lane: k, routing weight, this lane's chunk of row 0
    int kk[SLOTS];
    float wk[SLOTS];
    bool shs[SLOTS];  // this lane's slot i holds the shared expert
    const uint8_t* wrow[SLOTS];
    const uint16_t *srow[SLOTS], *brow[SLOTS];
    const int gi = (32 * li) / gsize;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
        const int k = i * EPI + sub;
        const int e = k < top_k ? eraw[i] : (k == top_k && nsh ? 0 : -1);
        shs[i] = SH && k == top_k;
        const gdsllm_affine_experts& p = shs[i] ? sdown : down;
        const bool valid = e >= 0 && e < p.num_experts;
        kk[i] = valid ? k : -1;
        wk[i] = valid ? (shs[i] ? 1.0f : h2f(wraw[i])) : 0.f;
        const int64_t ee = valid ? e : 0;
        wrow[i] = static_cast<const uint8_t*>(p.weight) + ee * p.weight_stride + 16 * li;
        srow[i] = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.scales) + ee * p.scale_stride) + gi;
        brow[i] = reinterpret_cast<const uint16_t*>(static_cast<const char*>(p.biases) + ee * p.bias_stride) + gi;
    }
    uint4 wv[R][SLOTS];
    uint32_t sv[R][SLOTS], bv[R][SLOTS];  // raw bits: see affine_rows
    // unconditional loads (see above): a slot without an expert reads expert
    // 0 and a row past the end reads the last row, both discarded
    auto issue = [&](int st) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int o0 = st * R + r;
            const int64_t o = o0 < H ? o0 : H - 1;
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                wv[r][i] = load_nt16(wrow[i] + o * (F / 2));
                sv[r][i] = srow[i][o * gpr];
                bv[r][i] = brow[i][o * gpr];
            }
        }
    };
    issue(gw);
    // prepared h records [top_k][CPR], one quarter (8 elements) per item
    bool h_nonfinite = false;
    {
        for (int base = 0; base < items; base += NT) {
            const int it = base + threadIdx.x;
            const bool live = it < items;
            const int wq = it & 3, c = (it >> 2) % CPR, k = (it >> 2) / CPR;
            float corr = 0.f, sum = 0.f;
            uint8_t* rec = smem + (k * CPR + c) * kRec;
            const int u = base / NT;
            if (live) {
                uint4 v;
                if (u < kEarly) {
                    v = hraw[0];
#pragma unroll
                    for (int e2 = 1; e2 < kEarly; ++e2)
                        if (u == e2) v = hraw[e2];
                } else {
                    v = *reinterpret_cast<const uint4*>(hbuf + k * F + 32 * c + 8 * wq);
                }
                xprep_quarter(rec, wq, v, corr, sum);
            }
            corr += __shfl_xor(corr, 1, 4);
            corr += __shfl_xor(corr, 2, 4);
            sum += __shfl_xor(sum, 1, 4);
            sum += __shfl_xor(sum, 2, 4);
            if (live && wq == 0) {
                *reinterpret_cast<float*>(rec + 64) = corr;
                *reinterpret_cast<float*>(rec + 68) = sum;
            }
            h_nonfinite |= live && !__builtin_isfinite(sum);
        }
    }
    const bool nonfinite = __syncthreads_or(h_nonfinite);
    if (T == 0) return;
    // combine of the routed sum v and the shared expert's vs for output row o
    auto combine_store = [&](int o, float v, float vs) {
        if constexpr (SH) {
            const float g = h2f(graw);
            const float sw = h2f(f2h_bits(fp32_rounded(1.0f / fp32_rounded(1.0f + expf(-g)))));
            const float sc = h2f(f2h_bits(fp32_rounded(sw * h2f(f2h_bits(vs)))));
            float r = h2f(f2h_bits(fp32_rounded(h2f(f2h_bits(v)) + sc)));
            if (r > 65504.0f) r = 65504.0f;  // NaN compares false both ways and stays NaN
            if (r < -65504.0f) r = -65504.0f;
            Y[o] = f2h_bits(r);
        } else {
            Y[o] = f2h_bits(v);
        }
    };
    if (nonfinite) {
        // the reference's per-element arithmetic: lane r < R takes row r of each stage
        wait_vmcnt<0>();
        for (int t = 0; t < T; ++t) {
            const int o = (gw + t * TW) * R + lane;
            if (lane < R && o < H)
                combine_store(o, moe_down_row_exact<false>(down, idx, rw, top_k, o, hbuf, false),
                              SH ? moe_down_row_exact<false>(sdown, idx, rw, top_k, o, hbuf, true) : 0.f);
        }
        return;
    }

    for (int t = 0; t < T; ++t) {
        const int st = gw + t * TW;
        uint4 cw[R][SLOTS];
        uint32_t cs[R][SLOTS], cb[R][SLOTS];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                cw[r][i] = wv[r][i];
                cs[r][i] = sv[r][i];
                cb[r][i] = bv[r][i];
            }
        if (t + 1 < T) issue(st + TW);
        float acc[R], accs[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = accs[r] = 0.f;
#pragma unroll
        for (int i = 0; i < SLOTS; ++i)
            if (kk[i] >= 0) {
                const uint8_t* rec = smem + (kk[i] * CPR + li) * kRec;
                uint32_t p[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint4 v = *reinterpret_cast<const uint4*>(rec + 16 * q);
                    p[4 * q] = v.x;
                    p[4 * q + 1] = v.y;
                    p[4 * q + 2] = v.z;
                    p[4 * q + 3] = v.w;
                }
                const float2 cs2 = *reinterpret_cast<const float2*>(rec + 64);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float d = chunk_dot_p(cw[r][i], p, cs2.x, cs2.y, h2f(cs[r][i]), h2f(cb[r][i]), nu);
                    if (SH && shs[i])
                        accs[r] += d;
                    else
                        acc[r] = __builtin_fmaf(wk[i], d, acc[r]);
                }
            }
        // sum over all 64 lanes (every expert slot and chunk); R = 2: lanes < 32 row 0
        auto lanes64 = [&](const float (&a)[R]) {
            float v;
            if constexpr (R == 2) {
                const bool h32 = lane & 32;
                v = (h32 ? a[1] : a[0]) + __shfl_xor(h32 ? a[0] : a[1], 32);
            } else {
                v = a[0] + __shfl_xor(a[0], 32);
            }
            v += __shfl_xor(v, 16);
            return lanes_sum<16>(v);
        };
        const float v = lanes64(acc);
        const int o = st * R + (R == 2 ? (lane >> 5) : 0);
        const bool writer = (lane & 31) == 0 && (R == 2 || lane == 0) && o < H;
        const float vs = SH ? lanes64(accs) : 0.f;
        if (writer) combine_store(o, v, vs);
    }
}

template <int LR, int CPL, int NB, class Rows>
int launch_affine_rows(const Rows& rows, const uint16_t* x, int K, int gsize, int64_t ldx, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(&affine_rows<LR, CPL, NB, Rows>);
    const int rps = (IsGateUp<Rows>::value ? 2 : 4) * (64 / LR);  // rows per stage, as in affine_rows
    const int stages = (rows.M + rps - 1) / rps;
    const int need = (stages + kWaves - 1) / kWaves;
    const int cap = blocks_per_cu(fn, 0, kThreads) * cu_count();
    const int grid = need < cap ? need : cap;
    const bool al16 = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (ldx % 8 == 0);
    hipLaunchKernelGGL((affine_rows<LR, CPL, NB, Rows>), dim3(grid), dim3(kThreads), 0, stream, rows, x, K, gsize, ldx,
                       al16 ? 1 : 0);
    return check_hip(hipGetLastError(), "affine_rows launch");
}

// Lanes per row LR and chunks per lane CPL for a row of `cpr` chunks;
// false when the row-span kernel does not cover the shape (CPL > 4).
bool rows_geometry(int cpr, int& lr, int& cpl) {
    lr = lanes_per_row(cpr);
    if (cpr < 8) return false;
    cpl = (cpr + lr - 1) / lr;
    return cpl <= 4;
}

template <int NB, class Rows>
int dispatch_rows(const Rows& rows, const uint16_t* x, int K, int gsize, int64_t ldx, hipStream_t stream) {
    int lr = 0, cpl = 0;
    rows_geometry(K / 32, lr, cpl);
    switch (lr * 8 + cpl) {
        case 64 * 8 + 1: return launch_affine_rows<64, 1, NB>(rows, x, K, gsize, ldx, stream);
        case 64 * 8 + 2: return launch_affine_rows<64, 2, NB>(rows, x, K, gsize, ldx, stream);
        case 64 * 8 + 3: return launch_affine_rows<64, 3, NB>(rows, x, K, gsize, ldx, stream);
        case 64 * 8 + 4: return launch_affine_rows<64, 4, NB>(rows, x, K, gsize, ldx, stream);
        case 32 * 8 + 1: return launch_affine_rows<32, 1, NB>(rows, x, K, gsize, ldx, stream);
        case 32 * 8 + 2: return launch_affine_rows<32, 2, NB>(rows, x, K, gsize, ldx, stream);
        case 16 * 8 + 1: return launch_affine_rows<16, 1, NB>(rows, x, K, gsize, ldx, stream);
        case 16 * 8 + 2: return launch_affine_rows<16, 2, NB>(rows, x, K, gsize, ldx, stream);
        case 8 * 8 + 1: return launch_affine_rows<8, 1, NB>(rows, x, K, gsize, ldx, stream);
        case 8 * 8 + 2: return launch_affine_rows<8, 2, NB>(rows, x, K, gsize, ldx, stream);
        default: return set_error(GDSLLM_ERR_UNSUPPORTED, "affine_rows: no kernel for this row length");
    }
}

// Workgroups of 16 waves (8 where 128 registers per lane would spill): every
// workgroup prepares all of h in LDS, so fewer, larger workgroups prepare it
// fewer times.
template <int LR, int SLOTS>
int launch_moe_down(const gdsllm_affine_experts& down, const int32_t* idx, const uint16_t* rw, const uint16_t* h,
                    int top_k, uint16_t* y, hipStream_t stream, const gdsllm_affine_experts* sdown = nullptr,
                    const uint16_t* gl = nullptr) {
    // 5 slots fit 1024 threads (128 registers) only without the shared
    // expert's accumulator
    constexpr int NT = (SLOTS <= 3 || SLOTS == 5) ? 1024 : 512;
    constexpr int NTS = SLOTS <= 3 ? 1024 : 512;
    const void* fn = sdown ? reinterpret_cast<const void*>(&moe_down_rows<LR, SLOTS, NTS, true>)
                           : reinterpret_cast<const void*>(&moe_down_rows<LR, SLOTS, NT, false>);
    const int nsh = sdown ? 1 : 0;
    const int nt = sdown ? NTS : NT;
    const size_t lds = static_cast<size_t>(top_k + nsh) * (down.in_dim / 32) * kRec;
    if (int rc = prepare_lds(fn, lds)) return rc;
    constexpr int R = SLOTS <= 4 ? 2 : 1;
    const int stages = static_cast<int>((down.out_dim + R - 1) / R);
    const int need = (stages + nt / 64 - 1) / (nt / 64);
    const int cap = blocks_per_cu(fn, lds, nt) * cu_count();
    const int grid = need < cap ? need : cap;
    if (sdown)
        hipLaunchKernelGGL((moe_down_rows<LR, SLOTS, NTS, true>), dim3(grid), dim3(NTS), lds, stream, down, idx, rw,
                           h, top_k, y, *sdown, gl);
    else
        hipLaunchKernelGGL((moe_down_rows<LR, SLOTS, NT, false>), dim3(grid), dim3(NT), lds, stream, down, idx, rw, h,
                           top_k, y, down, gl);
    return check_hip(hipGetLastError(), "moe_down_rows launch");
}

template <int LR>
int dispatch_moe_down_slots(int slots, const gdsllm_affine_experts& down, const int32_t* idx, const uint16_t* rw,
                            const uint16_t* h, int top_k, uint16_t* y, hipStream_t stream,
                            const gdsllm_affine_experts* sdown = nullptr, const uint16_t* gl = nullptr) {
    switch (slots) {
        case 1: return launch_moe_down<LR, 1>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        case 2: return launch_moe_down<LR, 2>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        case 3: return launch_moe_down<LR, 3>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        case 4: return launch_moe_down<LR, 4>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        case 5: return launch_moe_down<LR, 5>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        case 6: return launch_moe_down<LR, 6>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        case 7: return launch_moe_down<LR, 7>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        case 8: return launch_moe_down<LR, 8>(down, idx, rw, h, top_k, y, stream, sdown, gl);
        default: return set_error(GDSLLM_ERR_UNSUPPORTED, "moe_down_rows: too many expert slots");
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
    int lr = 0, cpl = 0;
    if (fast && batch <= 2 && rows_geometry(K / 32, lr, cpl)) {
        PlainRows rows{static_cast<const uint32_t*>(weight), static_cast<const uint16_t*>(scales),
                       static_cast<const uint16_t*>(biases), yp, ldy, M};
        const int rc = batch == 1 ? dispatch_rows<1>(rows, xp, K, g, ldx, s) : dispatch_rows<2>(rows, xp, K, g, ldx, s);
        return rc ? rc : ok();
    }
    const size_t budget = lds_budget();
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
    // fp16 gate/up outputs [top_k][2][F], then h [top_k][F]
    const size_t bytes = static_cast<size_t>(top_k) * 3 * static_cast<size_t>(ffn_dim) * 2;
    return (bytes + 255) / 256 * 256;
}

extern "C" size_t gdsllm_moe_step_workspace_size(int64_t top_k, int64_t ffn_dim) {
    return gdsllm_moe_gather_workspace_size(top_k + 1, ffn_dim) + 256;  // + the shared-gate logit
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

// ---- the same gather without a caller workspace ---------------------------------
// For callers that cannot allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid it): the gather's gate/up/h
// workspace is a fixed device array of kNoAllocScratchBytes instead.  Each
// device the library runs on holds its own copy of the array until the process
// ends; its address on a device is looked up once, with that device current,
// and cached.  Phase 1 writes every workspace entry phase 2 reads, so nothing
// is cleared and a call does not depend on what an earlier call left there.
// Calls that overlap on one device (several streams, several host threads)
// share the array and race: they must be ordered by the caller.
constexpr size_t kNoAllocScratchBytes = size_t(1) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kMaxScratchDevices];

// Device address of `scratch` on the current device.
static int scratch_on_current_device(void** out) {
    int dev = 0;
    if (int rc = check_hip(hipGetDevice(&dev), "moe_gather_affine_q4_noalloc: hipGetDevice")) return rc;
    if (dev < 0 || dev >= kMaxScratchDevices)
        return set_error(GDSLLM_ERR_UNSUPPORTED, "moe_gather_affine_q4_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                               "moe_gather_affine_q4_noalloc: hipGetSymbolAddress(scratch)"))
            return rc;
        if (!p) return set_error(GDSLLM_ERR_HIP, "moe_gather_affine_q4_noalloc: null scratch address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GDSLLM_OK;
}

// workspace == nullptr with fixed_ws: the fixed `scratch` array (looked up
// after every argument check, so a rejected call makes no HIP call).
static int moe_gather_impl(const std::string& n, const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                           const gdsllm_affine_experts* down, const void* x, const int32_t* idx,
                           const void* routing_weights, int64_t top_k, void* y, void* workspace,
                           size_t workspace_bytes, void* stream, bool fixed_ws = false) {
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
    if (!x || !idx || !routing_weights || !y || (!workspace && !fixed_ws))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 2 || reinterpret_cast<uintptr_t>(y) % 2 ||
        reinterpret_cast<uintptr_t>(routing_weights) % 2 || reinterpret_cast<uintptr_t>(idx) % 4 ||
        reinterpret_cast<uintptr_t>(workspace) % 16)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": misaligned pointer");
    if (workspace_bytes < gdsllm_moe_gather_workspace_size(top_k, F))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         n + (fixed_ws ? ": top_k * ffn too large for the fixed workspace (" : ": workspace too small (") +
                             std::to_string(gdsllm_moe_gather_workspace_size(top_k, F)) + " bytes needed, " +
                             std::to_string(workspace_bytes) + " available)");
    const size_t budget = lds_budget();
    const size_t lds1 = static_cast<size_t>(H / 32) * kRec, lds2 = static_cast<size_t>(top_k) * (F / 32) * kRec;
    if (lds1 > budget || lds2 > budget)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": hidden or top_k*ffn too large for LDS staging");
    if (fixed_ws)
        if (int rc = scratch_on_current_device(&workspace)) return rc;
    hipStream_t s = as_stream(stream);
    auto* gu = static_cast<uint16_t*>(workspace);
    const auto* xp = static_cast<const uint16_t*>(x);
    // Row-span path: hidden a multiple of 2048 up to 8192 (64 lanes per gate/up
    // row, <= 4 chunks each), ffn/32 in {16, 32, 64} lanes per down row and at
    // most 8 expert slots per lane.  Phase 1 writes g, u and h for every
    // selected slot (0 for an expert index out of range, which phase 2 skips),
    // so the workspace needs no clearing.
    const int cpr_h = static_cast<int>(H / 32), cpr_f = static_cast<int>(F / 32);
    const int slots = (cpr_f >= 16 && cpr_f <= 64) ? static_cast<int>((top_k + 64 / cpr_f - 1) / (64 / cpr_f)) : 0;
    const bool rows_path = H % 2048 == 0 && H <= 8192 && (cpr_f == 16 || cpr_f == 32 || cpr_f == 64) && slots >= 1 &&
                           slots <= 8 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (rows_path) {
        uint16_t* h = gu + top_k * 2 * F;
        GateUpPairs pairs{{}, *gate, *up, idx, gu, h, static_cast<int>(F), static_cast<int>(2 * top_k * F)};
        int rc;
        switch (cpr_h / 64) {
            case 1: rc = launch_affine_rows<64, 1, 1>(pairs, xp, static_cast<int>(H), static_cast<int>(gate->group_size), H, s); break;
            case 2: rc = launch_affine_rows<64, 2, 1>(pairs, xp, static_cast<int>(H), static_cast<int>(gate->group_size), H, s); break;
            case 3: rc = launch_affine_rows<64, 3, 1>(pairs, xp, static_cast<int>(H), static_cast<int>(gate->group_size), H, s); break;
            default: rc = launch_affine_rows<64, 4, 1>(pairs, xp, static_cast<int>(H), static_cast<int>(gate->group_size), H, s); break;
        }
        if (rc) return rc;
        const auto* wp = static_cast<const uint16_t*>(routing_weights);
        auto* yp = static_cast<uint16_t*>(y);
        const int tk = static_cast<int>(top_k);
        switch (cpr_f) {
            case 16: rc = dispatch_moe_down_slots<16>(slots, *down, idx, wp, h, tk, yp, s); break;
            case 32: rc = dispatch_moe_down_slots<32>(slots, *down, idx, wp, h, tk, yp, s); break;
            default: rc = dispatch_moe_down_slots<64>(slots, *down, idx, wp, h, tk, yp, s); break;
        }
        return rc ? rc : ok();
    }
    GateUpRows rows{*gate, *up, idx, gu, static_cast<int>(F), static_cast<int>(2 * top_k * F)};
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
    if (int rc = prepare_lds(fn, lds2)) return rc;
    const int passes = static_cast<int>((H + 64 / lr - 1) / (64 / lr));
    const int need = (passes + kWaves - 1) / kWaves;
    const int cap = blocks_per_cu(fn, lds2, kThreads) * cu_count();
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

extern "C" int gdsllm_moe_gather_affine_q4(const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                                           const gdsllm_affine_experts* down, const void* x, const int32_t* idx,
                                           const void* routing_weights, int64_t top_k, void* y, void* workspace,
                                           size_t workspace_bytes, void* stream) {
    return moe_gather_impl("moe_gather_affine_q4", gate, up, down, x, idx, routing_weights, top_k, y, workspace,
                           workspace_bytes, stream);
}

extern "C" size_t gdsllm_moe_gather_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int gdsllm_moe_gather_affine_q4_noalloc(const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                                                   const gdsllm_affine_experts* down, const void* x,
                                                   const int32_t* idx, const void* routing_weights, int64_t top_k,
                                                   void* y, void* stream) {
    return moe_gather_impl("moe_gather_affine_q4_noalloc", gate, up, down, x, idx, routing_weights, top_k, y, nullptr,
                           kNoAllocScratchBytes, stream, /*fixed_ws=*/true);
}

namespace {
// The routed step's extra inputs: the fp16 router logits of num_experts
// experts and where the picks and their weights go.
struct RouteArgs {
    const uint16_t* logits;
    int num_experts;
    int32_t* idx_out;
    uint16_t* w_out;
};
}  // namespace

// The fused decode step (gate/up with the shared expert, then down with the
// combine); route != null takes the picks from the router logits inside the
// gate/up launch (idx / routing_weights then name where they are stored).
static int moe_step_impl(const std::string& n, const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                         const gdsllm_affine_experts* down, const gdsllm_affine_experts* shared_gate,
                         const gdsllm_affine_experts* shared_up, const gdsllm_affine_experts* shared_down,
                         const void* x, const int32_t* idx, const void* routing_weights, int64_t top_k,
                         const void* shared_gate_weight, void* y, void* workspace, size_t workspace_bytes,
                         void* stream, const RouteArgs* route, bool dry_run = false) {
    std::string err;
    if (check_experts(gate, "gate", err) || check_experts(up, "up", err) || check_experts(down, "down", err) ||
        check_experts(shared_gate, "shared_gate", err) || check_experts(shared_up, "shared_up", err) ||
        check_experts(shared_down, "shared_down", err))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": " + err);
    if (top_k < 1 || top_k > 63)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": top_k must be in [1, 63], got " + std::to_string(top_k));
    const int64_t H = gate->in_dim, F = gate->out_dim;
    if (up->in_dim != H || up->out_dim != F || down->in_dim != F || down->out_dim != H ||
        gate->group_size != up->group_size || up->num_experts != gate->num_experts ||
        down->num_experts != gate->num_experts)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": gate/up [E,F,H] and down [E,H,F] shapes disagree");
    if (shared_gate->in_dim != H || shared_up->in_dim != H || shared_down->out_dim != H ||
        shared_gate->out_dim != shared_up->out_dim || shared_down->in_dim != shared_gate->out_dim)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": shared expert shapes disagree with hidden size");
    if (!x || !idx || !routing_weights || !shared_gate_weight || !y || !workspace)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 2 || reinterpret_cast<uintptr_t>(y) % 2 ||
        reinterpret_cast<uintptr_t>(routing_weights) % 2 || reinterpret_cast<uintptr_t>(shared_gate_weight) % 2 ||
        reinterpret_cast<uintptr_t>(idx) % 4 || reinterpret_cast<uintptr_t>(workspace) % 16)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": misaligned pointer");
    if (workspace_bytes < gdsllm_moe_step_workspace_size(top_k, F))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         n + ": workspace too small (" + std::to_string(workspace_bytes) + " < " +
                             std::to_string(gdsllm_moe_step_workspace_size(top_k, F)) + ")");
    // The fused step serves the row-span shapes with a shared expert of the
    // routed experts' width and grouping; anything else is the caller's
    // separate gather + shared expert + combine.
    const int cpr_h = static_cast<int>(H / 32), cpr_f = static_cast<int>(F / 32);
    const int nslot = static_cast<int>(top_k) + 1;
    const int slots = (cpr_f >= 16 && cpr_f <= 64) ? (nslot + 64 / cpr_f - 1) / (64 / cpr_f) : 0;
    const bool rows_path = H % 2048 == 0 && H <= 8192 && (cpr_f == 16 || cpr_f == 32 || cpr_f == 64) && slots >= 1 &&
                           slots <= 8 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                           reinterpret_cast<uintptr_t>(shared_gate_weight) % 16 == 0;
    if (!rows_path || shared_gate->out_dim != F || shared_gate->group_size != gate->group_size ||
        shared_up->group_size != gate->group_size || shared_down->group_size != down->group_size)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": shape outside the fused step (use the separate launches)");
    const size_t budget = lds_budget();
    if (static_cast<size_t>(nslot) * cpr_f * kRec > budget || static_cast<size_t>(cpr_h) * kRec > budget)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": hidden or (top_k+1)*ffn too large for LDS staging");
    if (dry_run) return GDSLLM_OK;
    hipStream_t s = as_stream(stream);
    auto* gu = static_cast<uint16_t*>(workspace);
    uint16_t* h = gu + static_cast<int64_t>(nslot) * 2 * F;  // after the gate/up outputs of every slot
    GateUpPairsShared pairs{};
    pairs.gate = *gate;
    pairs.up = *up;
    pairs.idx = idx;
    pairs.gu = gu;
    pairs.h = h;
    pairs.F = static_cast<int>(F);
    pairs.M = static_cast<int>(2 * nslot * F);
    pairs.sgate = *shared_gate;
    pairs.sup = *shared_up;
    pairs.shared_slot = static_cast<int>(top_k);
    // the logit sits after the gather's workspace
    auto* glw = reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(workspace) +
                                            gdsllm_moe_gather_workspace_size(top_k + 1, F));
    pairs.gate_w = static_cast<const uint16_t*>(shared_gate_weight);
    pairs.logit = glw;
    if (route) {
        pairs.route_logits = route->logits;
        pairs.route_e = route->num_experts;
        pairs.route_idx = route->idx_out;
        pairs.route_w = route->w_out;
    }
    const auto* xp = static_cast<const uint16_t*>(x);
    const int gs = static_cast<int>(gate->group_size);
    int rc;
    switch (cpr_h / 64) {
        case 1: rc = launch_affine_rows<64, 1, 1>(pairs, xp, static_cast<int>(H), gs, H, s); break;
        case 2: rc = launch_affine_rows<64, 2, 1>(pairs, xp, static_cast<int>(H), gs, H, s); break;
        case 3: rc = launch_affine_rows<64, 3, 1>(pairs, xp, static_cast<int>(H), gs, H, s); break;
        default: rc = launch_affine_rows<64, 4, 1>(pairs, xp, static_cast<int>(H), gs, H, s); break;
    }
    if (rc) return rc;
    const auto* wp = static_cast<const uint16_t*>(routing_weights);
    const uint16_t* gl = glw;
    auto* yp = static_cast<uint16_t*>(y);
    const int tk = static_cast<int>(top_k);
    switch (cpr_f) {
        case 16: rc = dispatch_moe_down_slots<16>(slots, *down, idx, wp, h, tk, yp, s, shared_down, gl); break;
        case 32: rc = dispatch_moe_down_slots<32>(slots, *down, idx, wp, h, tk, yp, s, shared_down, gl); break;
        default: rc = dispatch_moe_down_slots<64>(slots, *down, idx, wp, h, tk, yp, s, shared_down, gl); break;
    }
    return rc ? rc : ok();
}

extern "C" int gdsllm_moe_step_affine_q4(const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                                         const gdsllm_affine_experts* down, const gdsllm_affine_experts* shared_gate,
                                         const gdsllm_affine_experts* shared_up,
                                         const gdsllm_affine_experts* shared_down, const void* x, const int32_t* idx,
                                         const void* routing_weights, int64_t top_k, const void* shared_gate_weight,
                                         void* y, void* workspace, size_t workspace_bytes, void* stream) {
    return moe_step_impl("moe_step_affine_q4", gate, up, down, shared_gate, shared_up, shared_down, x, idx,
                         routing_weights, top_k, shared_gate_weight, y, workspace, workspace_bytes, stream, nullptr);
}

extern "C" size_t gdsllm_moe_step_routed_workspace_size(int64_t top_k, int64_t ffn_dim, int64_t num_experts) {
    const size_t logits = num_experts > 0 ? static_cast<size_t>(num_experts) * 2 : 0;
    return gdsllm_moe_step_workspace_size(top_k, ffn_dim) + (logits + 255) / 256 * 256;
}

extern "C" int gdsllm_moe_step_routed_affine_q4(const void* router_weight, const gdsllm_affine_experts* gate,
                                                const gdsllm_affine_experts* up, const gdsllm_affine_experts* down,
                                                const gdsllm_affine_experts* shared_gate,
                                                const gdsllm_affine_experts* shared_up,
                                                const gdsllm_affine_experts* shared_down, const void* x,
                                                int64_t top_k, const void* shared_gate_weight, void* y,
                                                int32_t* idx_out, void* weights_out, void* workspace,
                                                size_t workspace_bytes, void* stream) {
    const std::string n = "moe_step_routed_affine_q4";
    if (!gate) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": gate is null");
    const int64_t E = gate->num_experts, H = gate->in_dim, F = gate->out_dim;
    if (!router_weight || !idx_out || !weights_out || !workspace || !x)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (top_k < 1 || top_k > 63 || top_k > E)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": top_k must be in [1, min(63, num_experts)]");
    if (E > kRouteMaxExperts || E % 8 != 0 || H % 8 != 0)
        return set_error(GDSLLM_ERR_UNSUPPORTED,
                         n + ": routing inside the step takes num_experts <= 512, a multiple of 8, and hidden % 8 == 0");
    if (reinterpret_cast<uintptr_t>(router_weight) % 16 || reinterpret_cast<uintptr_t>(x) % 16 ||
        reinterpret_cast<uintptr_t>(idx_out) % 4 || reinterpret_cast<uintptr_t>(weights_out) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": misaligned pointer");
    const size_t step_ws = gdsllm_moe_step_workspace_size(top_k, F);
    if (workspace_bytes < gdsllm_moe_step_routed_workspace_size(top_k, F, E))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         n + ": workspace too small (" + std::to_string(workspace_bytes) + " < " +
                             std::to_string(gdsllm_moe_step_routed_workspace_size(top_k, F, E)) + ")");
    auto* logits = reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(workspace) + step_ws);
    const RouteArgs ra{logits, static_cast<int>(E), idx_out, static_cast<uint16_t*>(weights_out)};
    // every check of the step before the first launch
    if (int rc = moe_step_impl(n, gate, up, down, shared_gate, shared_up, shared_down, x, idx_out, weights_out, top_k,
                               shared_gate_weight, y, workspace, step_ws, stream, &ra, /*dry_run=*/true))
        return rc;
    // router logits: the fp16 GEMV that moe_route runs (gdsllm_gemv_f16), same bits
    if (int rc = gdsllm_gemv_f16(router_weight, x, logits, E, H, 1, H, E, stream)) return rc;
    return moe_step_impl(n, gate, up, down, shared_gate, shared_up, shared_down, x, idx_out, weights_out, top_k,
                         shared_gate_weight, y, workspace, step_ws, stream, &ra);
}
