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

#include <algorithm>
#include <type_traits>
#include <utility>

#include "common.h"

namespace gdsllm {
namespace {

enum class Fmt { Q4_0, Q8_0 };

// Exact products: every weight pair enters the dot products as its exact value
// (q - 8 for Q4_0, q for Q8_0: the exponent-trick pair minus its bias, exact
// in packed fp16), so each product w*x is the reference's product and the fp32
// sum has the reference's magnitude; no offset correction is subtracted.
// Without it the sum runs over (1024 + q)*x and the correction c cancels it
// afterwards, which loses about 10 bits to cancellation when one x dwarfs the
// rest (an activation near 65504 against N(0, 1)) and turns an infinite x into
// inf - inf = NaN on every row (the reference gives +-inf, NaN only where the
// weight is 0).  The exact form costs one packed subtract per weight pair
// (about 4% at 11008x4096, batch 1), so a window takes it only when its x calls
// for it (load_slice); kRowsExact = false disables it (measurement only).
// The batched kernels take the exact form always: the staged kernel
// (kStagedExact), a fallback, and the Q4_0 MFMA kernels (kCodesExact), where
// the weight operand is unbiased the same way and the offset-correction MFMAs
// drop out (deciding per wave from its slice of x, as the row-span kernel
// does per window, measured no faster on the x-in-registers kernel).
constexpr bool kRowsExact = true;
constexpr bool kStagedExact = true;
constexpr bool kCodesExact = true;

// (a - bias) on both fp16 halves (v_pk_add_f16; exact for the pairs below).
__device__ __forceinline__ uint32_t unbias_pair(uint32_t a, uint32_t neg_bias_pair) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, a) + __builtin_bit_cast(half2_t, neg_bias_pair));
}
constexpr uint32_t kNeg1032 = 0xE408E408u;  // fp16 -1032 in both halves
constexpr uint32_t kNeg72 = 0xD480D480u;    // -72
constexpr uint32_t kNeg1152 = 0xE480E480u;  // -1152

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
                uint32_t p0 = nib_lo_pair(v), p1 = nib_hi_pair(v);
                uint32_t p2 = nib_lo_pair(vs), p3 = nib_hi_pair(vs);
                if constexpr (kStagedExact) {
                    p0 = unbias_pair(p0, kNeg1032), p1 = unbias_pair(p1, kNeg72);
                    p2 = unbias_pair(p2, kNeg1032), p3 = unbias_pair(p3, kNeg72);
                }
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
                uint32_t p0 = (u0 & 0x00FF00FFu) | 0x64006400u;
                uint32_t p1 = ((u0 >> 8) & 0x00FF00FFu) | 0x64006400u;
                uint32_t p2 = (u1 & 0x00FF00FFu) | 0x64006400u;
                uint32_t p3 = ((u1 >> 8) & 0x00FF00FFu) | 0x64006400u;
                if constexpr (kStagedExact) {
                    p0 = unbias_pair(p0, kNeg1152), p1 = unbias_pair(p1, kNeg1152);
                    p2 = unbias_pair(p2, kNeg1152), p3 = unbias_pair(p3, kNeg1152);
                }
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
            if constexpr (kStagedExact) {
                acc[b] = __builtin_fmaf(d, Sd[b], acc[b]);
            } else {
                const float corr = *reinterpret_cast<const float*>(xrec0 + b * rec_stride + 512 + 4 * i);
                acc[b] = __builtin_fmaf(d, Sd[b] - corr, acc[b]);
            }
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

// ---- row-span kernel (batch 1..2) ----------------------------------------------
// Stages of 4 rows x one window of 16 super-blocks (128 blocks), moved from
// HBM straight into a per-wave LDS buffer by 16-byte-per-lane DMA transfers
// (no staging registers, no LDS store instructions); from there lane c owns
// blocks 2c and 2c+1 of the window in all 4 rows.  A stage is consumed in two
// halves, rows 0-1 as soon as the transfers holding them have retired, and
// with two buffers per wave the next stage is in flight meanwhile.  The lane's
// slice of x (blocks 2c, 2c+1 of the window: 64 elements per batch row) is the
// same for every row it touches, so it sits in registers, permuted once per
// window into the pair order the unpacked nibbles come out in, with each
// block's offset correction.  The 4 (row, block) chains of a
// half stage are interleaved, and the 4 row sums of a wave reduce in 3
// cross-lane swaps + 4 DPP steps.

constexpr int kWinBlocks = kSbPerWindow * 8;  // blocks per row in one stage

// fp16 pairs (c, c): 1032 = 1024 + 8 and 72 = 64 + 8 undo the exponent-trick
// bias and the Q4_0 offset 8 of low / high nibbles; 1152 = 1024 + 128 undoes
// the biased Q8_0 byte.
constexpr uint32_t kPair1032 = 0x64086408u;
constexpr uint32_t kPair72 = 0x54805480u;
constexpr uint32_t kPair1152 = 0x64806480u;

// (lo, hi) = low halves / high halves of (u, v): v_perm_b32 selectors with
// S0 = v, S1 = u.
constexpr uint32_t kSelLo = 0x05040100u;
constexpr uint32_t kSelHi = 0x07060302u;


// A lane's x slice: fp16 pairs of blocks 2c, 2c+1 of the window in the order
// the unpacked nibbles come out in (p[b][k]: block k), and each block's offset
// correction: 1032*sum(x[0..16)) + 72*sum(x[16..32)) (Q4_0) or 1152*sum(x)
// (Q8_0), so a block reduces to d * (S - c).
template <int NB>
struct XSlice {
    uint32_t p[NB][2][16];
    float c[NB][2];
    bool exact;  // wave-uniform: this window's x needs the exact products
};

// 32 raw fp16 of one block (r[i] = elements 2i, 2i+1) -> 16 pairs in unpack
// order and the block's offset correction (returned).
template <Fmt F>
__device__ __forceinline__ float permute_block(const uint32_t* r, uint32_t* p) {
    float c = 0.f;
    if constexpr (F == Fmt::Q4_0) {
        // qs dword dd: low nibbles = elements 4dd..4dd+3, high = 16+4dd..19+4dd;
        // pairs (bytes 0,2 low) (bytes 0,2 high) (bytes 1,3 low) (bytes 1,3 high)
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) {
            const uint32_t u = r[2 * dd], v = r[2 * dd + 1];
            const uint32_t uh = r[8 + 2 * dd], vh = r[9 + 2 * dd];
            p[4 * dd + 0] = __builtin_amdgcn_perm(v, u, kSelLo);
            p[4 * dd + 1] = __builtin_amdgcn_perm(vh, uh, kSelLo);
            p[4 * dd + 2] = __builtin_amdgcn_perm(v, u, kSelHi);
            p[4 * dd + 3] = __builtin_amdgcn_perm(vh, uh, kSelHi);
            c = dot2(u, kPair1032, c);
            c = dot2(v, kPair1032, c);
            c = dot2(uh, kPair72, c);
            c = dot2(vh, kPair72, c);
        }
    } else {
        // qs dword dd = elements 4dd..4dd+3: pairs (bytes 0,2) (bytes 1,3)
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
            const uint32_t u = r[2 * dd], v = r[2 * dd + 1];
            p[2 * dd] = __builtin_amdgcn_perm(v, u, kSelLo);
            p[2 * dd + 1] = __builtin_amdgcn_perm(v, u, kSelHi);
            c = dot2(u, kPair1152, c);
            c = dot2(v, kPair1152, c);
        }
    }
    return c;
}

// Raw x in LDS, laid out for the slices: record (b, w) = batch row b, window w
// is 8 KiB; its 16-byte slot 64i + c holds elements [64c + 8i, 64c + 8i + 8)
// of the window, so reading chunk i of every lane's slice is one
// conflict-free 1 KiB row.  The workgroup fills it with DMA transfers (slot
// row i of record (b, w) = transfer (b*NW + w)*8 + i), which the compiler
// does not count when it waits for an ordinary load issued before them: x
// loaded into registers ahead of the weight transfers would wait for all of
// them.
__host__ __device__ inline int rows_xraw_bytes(int nb, int nw) { return nb * nw * 8192; }

template <int NB>
__device__ __forceinline__ void rows_xraw_issue(uint8_t* xraw, const uint16_t* __restrict__ X, int64_t ldx, int K,
                                                int NW, int wave, int wpg, int lane) {
    const int n = NB * NW * 8;
    for (int t = wave; t < n; t += wpg) {
        const int i = t & 7, w = (t >> 3) % NW, b = (t >> 3) / NW;
        const int e = 4096 * w + 64 * lane + 8 * i;  // first element of the slot
        dma16_cached(e < K ? X + b * ldx + e : X, xraw + 1024 * t);
    }
}

// The slice of window w, read with the raw LDS helpers (no weight transfer
// ever targets the x region), permuted into unpack order, with corrections.
//
// It also decides, for the whole wave, whether this window takes the exact
// products (see kRowsExact): when some block of x holds a quarter or more of
// the window's energy sum(x^2) of its batch row, or any energy is not finite
// (an infinite or NaN x).  Below that share the offset-corrected sum stays
// within 2e-4 of ||w * x|| per block (its error is about 2^-22 * 1032 *
// sum|x| of the block, and sum|x| <= sqrt(32 * E / 4)); activations drawn
// from one distribution never come near it, an outlier column does.
template <Fmt F, int NB>
__device__ __forceinline__ void load_slice(XSlice<NB>& xs, const uint8_t* xraw, int NW, int w, int K, int lane) {
    u32x4_t v[NB][8];
#pragma unroll
    for (int b = 0; b < NB; ++b) lds_read16x8_sync(lds_addr(xraw + (b * NW + w) * 8192 + 16 * lane), v[b]);
    // lane's two blocks lie inside in_dim (filler x past the end is ignored)
    const bool valid = 4096 * w + 64 * lane < K;
    bool risky = false;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        float e[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            uint32_t r[16];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) r[4 * i + j] = v[b][4 * k + i][j];
            xs.c[b][k] = permute_block<F>(r, xs.p[b][k]);
            float en = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) en = dot2(r[i], r[i], en);
            e[k] = valid ? en : 0.f;
        }
        // window energy of batch row b in every lane: lane-half swaps, then the 16-lane DPP sum
        float tot = swap_sum32(e[0] + e[1], e[0] + e[1]);
        tot = row16_sum(swap_sum16(tot, tot));
#pragma unroll
        for (int k = 0; k < 2; ++k) risky |= !(e[k] <= 0.f) && !(4.f * e[k] < tot);
    }
    xs.exact = kRowsExact && __builtin_amdgcn_ballot_w64(risky) != 0;
}


// Adds the dot products of qs dword dd of one block with its x pairs to S.
template <Fmt F, bool EXACT>
__device__ __forceinline__ float dword_dot(uint32_t q, const uint32_t* xp, int dd, float S, const NibUnpack& nu) {
    if constexpr (F == Fmt::Q4_0) {
        const uint32_t vs = q >> 8;
        if constexpr (EXACT) {
            S = dot2(unbias_pair(nu.lo_c(q), kNeg1032), xp[4 * dd + 0], S);
            S = dot2(unbias_pair(nu.hi_c(q), kNeg72), xp[4 * dd + 1], S);
            S = dot2(unbias_pair(nu.lo_c(vs), kNeg1032), xp[4 * dd + 2], S);
            S = dot2(unbias_pair(nu.hi_c(vs), kNeg72), xp[4 * dd + 3], S);
        } else {
            S = dot2(nu.lo_c(q), xp[4 * dd + 0], S);
            S = dot2(nu.hi_c(q), xp[4 * dd + 1], S);
            S = dot2(nu.lo_c(vs), xp[4 * dd + 2], S);
            S = dot2(nu.hi_c(vs), xp[4 * dd + 3], S);
        }
    } else {
        // biased byte u = q + 128 in the low byte of each half: 1024 + u
        const uint32_t u = q ^ 0x80808080u;
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04020400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030401u);
        S = dot2(EXACT ? unbias_pair(p0, kNeg1152) : p0, xp[2 * dd], S);
        S = dot2(EXACT ? unbias_pair(p1, kNeg1152) : p1, xp[2 * dd + 1], S);
    }
    return S;
}

// Sums acc[0..3] over the 64 lanes of the wave.  Lane L ends up holding the
// total of row L >> 4: lanes 0-15 row 0, 16-31 row 1, 32-47 row 2, 48-63 row 3
// (two lane-half swaps, then the 16-lane DPP sum).
__device__ __forceinline__ float reduce_rows4(const float (&acc)[4]) {
    const float k02 = swap_sum32(acc[0], acc[2]);  // rows 0 | 2 over lanes l, l+32
    const float k13 = swap_sum32(acc[1], acc[3]);  // rows 1 | 3
    return row16_sum(swap_sum16(k02, k13));
}

// Where a row-span launch reads weights and writes results.  Plain: up to 4
// matrices of the same in_dim sharing x, each served by its own range of
// workgroups (gb_end); row r of matrix m for batch row b goes to
// y[m][b*ldy[m] + r].  Gate/up pairing: w[0] = gate, w[1] = up,
// both m[0] rows; row group g holds gate rows 2g, 2g+1 (stage rows 0-1) and up
// rows 2g, 2g+1 (stage rows 2-3), and y[0][b*ldy[0] + r] receives
// h = fp16(silu(fp16 gate) * fp16 up), the SwiGLU input of the down projection.
constexpr int kMaxGroup = 4;
struct RowsTarget {
    const uint8_t* w[kMaxGroup];
    uint16_t* y[kMaxGroup];
    int64_t ldy[kMaxGroup];
    int m[kMaxGroup];
    int gb_end[kMaxGroup];  // groups: workgroups [gb_end[i-1], gb_end[i]) serve matrix i
    int n;
    // 1: a wave issues its next stage after consuming the whole current one
    // (waves that share a SIMD); 0: rows 0-1's slots as soon as they are read
    int late_issue;
};

// One stage: stage row 0 of window super-block sb0 starts at base0 (pairing:
// rows 0-1 at base0, rows 2-3 at base1), nrows valid rows (per matrix when
// paired), nsb super-blocks.
struct RowsStage {
    const uint8_t* base0;
    const uint8_t* base1;
    uint16_t* y;
    int64_t ldy;
    int r0, nrows, nsb, seg_chunks;
};

// The fields of this workgroup's matrix (pair), copied once into SGPRs (an
// empty asm pins them there; otherwise the compiler re-reads the kernel
// argument inside the loop and waits for it).  first_block/blocks: this
// matrix's workgroup range.
struct TargetRegs {
    const uint8_t *w0, *w1;
    uint16_t* y;
    int64_t ldy;
    int m, first_block, blocks;
    // MODE 0: one matrix; 1: a group (matrix chosen by workgroup); 2: gate/up.
    template <int MODE>
    __device__ __forceinline__ void load(const RowsTarget& tg) {
        if constexpr (MODE != 1) {
            w0 = tg.w[0], w1 = MODE == 2 ? tg.w[1] : tg.w[0], y = tg.y[0], ldy = tg.ldy[0], m = tg.m[0];
            first_block = 0;
            blocks = gridDim.x;
        } else {
            const int bx = blockIdx.x;
            const int i = (tg.n > 1 && bx >= tg.gb_end[0]) + (tg.n > 2 && bx >= tg.gb_end[1]) +
                          (tg.n > 3 && bx >= tg.gb_end[2]);
            switch (i) {
                case 0: w0 = tg.w[0], y = tg.y[0], ldy = tg.ldy[0], m = tg.m[0], first_block = 0; break;
                case 1: w0 = tg.w[1], y = tg.y[1], ldy = tg.ldy[1], m = tg.m[1], first_block = tg.gb_end[0]; break;
                case 2: w0 = tg.w[2], y = tg.y[2], ldy = tg.ldy[2], m = tg.m[2], first_block = tg.gb_end[1]; break;
                default: w0 = tg.w[3], y = tg.y[3], ldy = tg.ldy[3], m = tg.m[3], first_block = tg.gb_end[2]; break;
            }
            blocks = (i == 0 ? tg.gb_end[0] : i == 1 ? tg.gb_end[1] : i == 2 ? tg.gb_end[2] : tg.gb_end[3]) -
                     first_block;
            w1 = w0;
        }
        asm volatile("" : "+s"(w0), "+s"(w1), "+s"(y), "+s"(ldy), "+s"(m), "+s"(first_block), "+s"(blocks));
    }
};

template <Fmt F, bool PAIRED>
__device__ __forceinline__ RowsStage rows_stage(const TargetRegs& tg, int rg, int win, int S, uint32_t row_bytes) {
    using L = Layout<F>;
    RowsStage st;
    const int sb0 = win * kSbPerWindow;
    st.nsb = min(kSbPerWindow, S - sb0);
    st.seg_chunks = st.nsb * L::kSbChunks;
    const int64_t col = static_cast<int64_t>(sb0) * L::kSbBytes;
    st.r0 = (PAIRED ? 2 : kRowsPerStage) * rg;
    st.nrows = min(PAIRED ? 2 : kRowsPerStage, tg.m - st.r0);
    st.base0 = tg.w0 + st.r0 * static_cast<int64_t>(row_bytes) + col;
    st.base1 = tg.w1 + st.r0 * static_cast<int64_t>(row_bytes) + col;
    st.y = tg.y;
    st.ldy = tg.ldy;
    return st;
}

// Stage transfers, global memory straight to LDS.  Slot s = 64j + lane of a
// wave's stage buffer (bytes [16s, 16s+16)) holds chunk s % kSegChunks of the
// stage's row s / kSegChunks, so the rows of a stage sit kSegBytes apart in LDS
// whatever its width.  A full stage (16 super-blocks, every row valid) has the
// same per-lane offsets every time (goff, computed once; with pairing, bit 31
// selects base1); a partial one (the last rows, the last window of a row)
// points the slots it does not cover at its first chunk.  `live == false`
// sends every slot to the first 16 bytes of x, a dummy transfer that keeps
// each wave's count of transfers fixed.  Transfers [J0, J1) of the stage;
// offsets stay in 32 bits: in_dim <= 2^20.
template <Fmt F, int J0, int J1, bool PAIRED>
__device__ __forceinline__ void rows_issue(uint8_t* buf, const RowsStage& st, const void* dummy, uint32_t row_bytes,
                                           const uint32_t (&goff)[Layout<F>::kSbChunks], bool live, int lane) {
    using L = Layout<F>;
    constexpr int kSegChunks = kSbPerWindow * L::kSbChunks;
    if (!live) {
#pragma unroll
        for (int j = J0; j < J1; ++j) dma16(dummy, buf + 1024 * j);
    } else if (st.nrows == (PAIRED ? 2 : kRowsPerStage) && st.nsb == kSbPerWindow) {
#pragma unroll
        for (int j = J0; j < J1; ++j) {
            if constexpr (PAIRED)
                dma16(((goff[j] >> 31) ? st.base1 : st.base0) + (goff[j] & 0x7FFFFFFFu), buf + 1024 * j);
            else
                dma16(st.base0 + goff[j], buf + 1024 * j);
        }
    } else {
#pragma unroll
        for (int j = J0; j < J1; ++j) {
            const uint32_t s = 64 * j + lane;
            const uint32_t rl = s / kSegChunks, off = s - rl * kSegChunks;
            const uint32_t rr = PAIRED ? (rl & 1) : rl;  // row within its matrix
            const bool in = rr < static_cast<uint32_t>(st.nrows) && off < static_cast<uint32_t>(st.seg_chunks);
            const uint8_t* base = (PAIRED && rl >= 2) ? st.base1 : st.base0;
            dma16(base + (in ? __umul24(rr, row_bytes) + 16 * off : 0u), buf + 1024 * j);
        }
    }
}

// LDS of the row-span kernel (all dynamic): one stage buffer per wave, then raw x.
template <Fmt F, int NB>
size_t rows_lds_bytes(int nw, int wpg) {
    return static_cast<size_t>(wpg) * stage_bytes<F>() + static_cast<size_t>(rows_xraw_bytes(NB, nw));
}

// Rows R0 .. R0+NR-1 of a stage in LDS: lane c's blocks 2c, 2c+1 of each row
// against its x slice, added to acc[b][R0+r].  The NR rows x 2 blocks x NB
// dot-product chains interleave.
template <Fmt F, int NB, int R0, int NR, bool EXACT>
__device__ __forceinline__ void rows_pair_impl(const uint8_t* buf, const XSlice<NB>& xs, float (&acc)[NB][4],
                                               const NibUnpack& nu, int lane) {
    using L = Layout<F>;
    constexpr int kSegBytes = kSbPerWindow * L::kSbBytes;
    constexpr int kSpanDw = L::kBlockBytes / 2;  // dwords of a lane's 2 blocks
    constexpr int kQd = (L::kBlockBytes - 2) / 4;  // qs dwords per block
    uint32_t D[NR][kSpanDw];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(buf + (R0 + r) * kSegBytes) + kSpanDw * lane;
#pragma unroll
        for (int i = 0; i < kSpanDw; ++i) D[r][i] = src[i];
    }
    // block 2c: scale = bytes 0-1, qs from byte 2; block 2c+1 starts at byte
    // kBlockBytes (dword-aligned halfway point: scale in the high half)
    float Sx[NB][NR][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < NR; ++r) Sx[b][r][0] = Sx[b][r][1] = 0.f;
#pragma unroll
    for (int dd = 0; dd < kQd; ++dd)
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const uint32_t q0 = align2(D[r][dd], D[r][dd + 1]);
            const uint32_t q1 = D[r][kQd + 1 + dd];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                Sx[b][r][0] = dword_dot<F, EXACT>(q0, xs.p[b][0], dd, Sx[b][r][0], nu);
                Sx[b][r][1] = dword_dot<F, EXACT>(q1, xs.p[b][1], dd, Sx[b][r][1], nu);
            }
        }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float d0 = h2f(D[r][0] & 0xFFFFu), d1 = h2f(D[r][kQd] >> 16);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if constexpr (EXACT) {
                acc[b][R0 + r] = __builtin_fmaf(d0, Sx[b][r][0], acc[b][R0 + r]);
                acc[b][R0 + r] = __builtin_fmaf(d1, Sx[b][r][1], acc[b][R0 + r]);
            } else {
                acc[b][R0 + r] = __builtin_fmaf(d0, Sx[b][r][0] - xs.c[b][0], acc[b][R0 + r]);
                acc[b][R0 + r] = __builtin_fmaf(d1, Sx[b][r][1] - xs.c[b][1], acc[b][R0 + r]);
            }
        }
    }
}

// Rows of `target` times x (MODE 0: one matrix; 1: a group; 2: gate/up pairs); x must be 16-byte aligned
// with ldx % 8 == 0.  Workgroups of kWaves waves; LDS (dynamic): the waves'
// stage buffers, then raw x.  One buffer per wave: after rows 0-1 of a stage are consumed, the next
// stage's transfers that land in their slots only (kEarly) are issued, the
// rest after rows 2-3.
//
// SW (split windows, MODE 0, in_dim over NW >= 2 windows of 4096): wave w
// takes window w % NW of row-group slot w / NW (WV = NW x slots), so the NW
// stages of a row group stream at once from NW waves instead of one after
// another from one.  Each stage's four row sums go to a partial area after
// x, [stage t][wave][batch row][4]; after a workgroup barrier the window-0
// waves add the NW partials of each row in window order and store y.
template <Fmt F, int NB, int MODE, int WV = kWaves, bool SW = false>
__global__ __launch_bounds__(WV * 64) void gguf_gemv_rows(const RowsTarget target, const uint16_t* __restrict__ X,
                                                          int K, int64_t ldx) {
    constexpr bool PAIRED = MODE == 2;
    using L = Layout<F>;
    constexpr int C = L::kSbChunks;                        // transfers per stage
    constexpr int kSegChunks = kSbPerWindow * L::kSbChunks;
    // transfers (of 64 16-byte chunks) that complete stage rows 0 .. r
    constexpr int kRowDone[4] = {(kSegChunks + 63) / 64, (2 * kSegChunks + 63) / 64, (3 * kSegChunks + 63) / 64, C};
    constexpr int kEarly = (2 * kSegChunks) / 64;          // transfers within rows 0-1 only
    static_assert(C - kRowDone[2] + kEarly < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int S = K >> 8;
    const uint32_t row_bytes = static_cast<uint32_t>(S) * L::kSbBytes;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    uint8_t* buf = lds + wave * stage_bytes<F>();
    uint8_t* xp = lds + WV * stage_bytes<F>();
    const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();
    TargetRegs tg;
    tg.load<MODE>(target);
    const int RG = (tg.m + (PAIRED ? 1 : kRowsPerStage - 1)) / (PAIRED ? 2 : kRowsPerStage);
    const int NW = (S + kSbPerWindow - 1) / kSbPerWindow;
    static_assert(!SW || MODE == 0, "split windows serve one matrix");
    // plain: wave gw takes row groups gw, gw + total_waves, ..., each window
    // in turn; SW: wave (slot, my_win) takes window my_win of row groups
    // rg0, rg0 + total_slots, ...
    const int R = SW ? WV / NW : 1;  // row-group slots per workgroup
    const int my_win = SW ? wave % NW : 0;
    const int total_waves = tg.blocks * WV, total_slots = tg.blocks * R;
    const int gw = SW ? (blockIdx.x - tg.first_block) * R + wave / NW : (blockIdx.x - tg.first_block) * WV + wave;
    const int my_rgs = gw < RG ? (RG - 1 - gw) / (SW ? total_slots : total_waves) + 1 : 0;
    const int T = SW ? my_rgs : my_rgs * NW;
    const NibUnpack nu;
    auto stage_at = [&](int t) {
        if constexpr (SW) return rows_stage<F, PAIRED>(tg, gw + t * total_slots, my_win, S, row_bytes);
        else return rows_stage<F, PAIRED>(tg, gw + (t / NW) * total_waves, t % NW, S, row_bytes);
    };
    const uint32_t part0 = lds_addr(xp + rows_xraw_bytes(NB, NW));  // SW: the partial row sums

    uint32_t goff[C];
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const uint32_t c = 64 * j + lane;
        const uint32_t rl = c / kSegChunks;
        const uint32_t rr = PAIRED ? (rl & 1) : rl;
        goff[j] = ((PAIRED && rl >= 2) ? 0x80000000u : 0u) | (rr * row_bytes + 16 * (c - rl * kSegChunks));
    }

    // Request order: raw x, then the first stage of weights (always issued,
    // dummy when the wave has no stage); waiting for all but the weight
    // transfers then waits for x only.  A compute unit returns its requests in
    // order, so every wave's x is requested before any wave's weights.
    // The stage goes out in two parts, rows 0-1 before the wave prepares its
    // x slice and rows 2-3 after: once the compute unit's request queue is
    // full a transfer instruction waits for room, and the slice (~110 VALU
    // instructions) is then prepared while rows 0-1 travel instead of after
    // the whole stage has been queued.
    // Top wave priority while x is issued: x requests of a workgroup that
    // starts next to running ones leave ahead of their weight requests
    // (11008x4096 at batch 1: 7.006 against 7.038 us per call).
    __builtin_amdgcn_s_setprio(3);
    rows_xraw_issue<NB>(xp, X, ldx, K, NW, wave, WV, lane);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_s_setprio(0);
    constexpr int kJ = kRowDone[1];
    const RowsStage st0 = stage_at(0);
    rows_issue<F, 0, kJ, PAIRED>(buf, st0, X, row_bytes, goff, T > 0, lane);
    wait_vmcnt<kJ>();
    lds_barrier();  // every wave's share of x has landed
    {
        // Waves whose transfers went out late (the queue was full) hold the
        // last data of the launch: they get the SIMD first from here on,
        // graded by how late (s_memrealtime counts at 100 MHz).  11008 x
        // 4096 at batch 1: 7.01 -> 6.71 us per call.
        const uint64_t dt = __builtin_amdgcn_s_memrealtime() - t_entry;
        if (dt > 300) __builtin_amdgcn_s_setprio(3);
        else if (dt > 200) __builtin_amdgcn_s_setprio(2);
        else if (dt > 100) __builtin_amdgcn_s_setprio(1);
    }

    XSlice<NB> xs;
    if (T > 0) load_slice<F, NB>(xs, xp, NW, my_win, K, lane);
    rows_issue<F, kJ, C, PAIRED>(buf, st0, X, row_bytes, goff, T > 0, lane);
    int xwin = my_win;
    float acc[NB][4];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[b][r] = 0.f;

    for (int t = 0; t < T; ++t) {
        const int win = SW ? my_win : t % NW;
        const RowsStage st = stage_at(t);
        const bool next = t + 1 < T;
        if (win != xwin) {
            load_slice<F, NB>(xs, xp, NW, win, K, lane);
            xwin = win;
        }
        // Lanes past the end of a partial window skip; rows past M compute on
        // filler bytes and are never stored.  In flight here: this stage only.
        // Each row is consumed as soon as the transfers that hold it retire.
        // The window's product form is one wave-uniform branch around the whole
        // stage, so each form is straight-line code the compiler schedules
        // across rows.
        const bool active = lane < st.nsb * 4;
        const RowsStage nx = stage_at(t + 1);
        auto consume = [&](auto exact_c, auto late_c) {
            constexpr bool EX = decltype(exact_c)::value;
            wait_vmcnt<C - kRowDone[0]>();
            if (active) rows_pair_impl<F, NB, 0, 1, EX>(buf, xs, acc, nu, lane);
            wait_vmcnt<C - kRowDone[1]>();
            if (active) rows_pair_impl<F, NB, 1, 1, EX>(buf, xs, acc, nu, lane);
            if constexpr (decltype(late_c)::value) {
                // the next stage goes out once this one is read: a wave that
                // would wait for room in the request queue does so after its
                // products (7B gate/up and lm_head: 11.7 -> 11.3 and 13.9 ->
                // 13.7 us; the 4096 x 11008 down projection, one wave per
                // SIMD, is faster with the early refill)
                wait_vmcnt<C - kRowDone[2]>();
                if (active) rows_pair_impl<F, NB, 2, 1, EX>(buf, xs, acc, nu, lane);
                wait_vmcnt<0>();
                if (active) rows_pair_impl<F, NB, 3, 1, EX>(buf, xs, acc, nu, lane);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (next) rows_issue<F, 0, C, PAIRED>(buf, nx, X, row_bytes, goff, true, lane);
                return;
            }
            // refill slots of rows 0-1 once their reads have returned
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (next) {
                rows_issue<F, 0, kEarly, PAIRED>(buf, nx, X, row_bytes, goff, true, lane);
                wait_vmcnt<C - kRowDone[2] + kEarly>();
                if (active) rows_pair_impl<F, NB, 2, 1, EX>(buf, xs, acc, nu, lane);
                wait_vmcnt<kEarly>();
            } else {
                wait_vmcnt<C - kRowDone[2]>();
                if (active) rows_pair_impl<F, NB, 2, 1, EX>(buf, xs, acc, nu, lane);
                wait_vmcnt<0>();
            }
            if (active) rows_pair_impl<F, NB, 3, 1, EX>(buf, xs, acc, nu, lane);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (next) rows_issue<F, kEarly, C, PAIRED>(buf, nx, X, row_bytes, goff, true, lane);
        };
        if (target.late_issue) {
            if (kRowsExact && xs.exact) consume(std::true_type{}, std::true_type{});
            else consume(std::false_type{}, std::true_type{});
        } else {
            if (kRowsExact && xs.exact) consume(std::true_type{}, std::false_type{});
            else consume(std::false_type{}, std::false_type{});
        }
        if constexpr (SW) {
            // this window's four row sums; written with raw LDS stores (a
            // compiler-visible one would wait for the transfers in flight)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float v = reduce_rows4(acc[b]);
                if ((lane & 15) == 0)
                    lds_write4_raw(part0 + 4u * (((t * WV + wave) * NB + b) * 4 + (lane >> 4)),
                                   __builtin_bit_cast(uint32_t, v));
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[b][r] = 0.f;
            }
        } else if (win == NW - 1) {
            const int row = lane >> 4;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float v = reduce_rows4(acc[b]);
                if constexpr (PAIRED) {
                    // lanes 0-31: gate rows r0, r0+1 in g, the matching up rows in u
                    float g = v, u = v;
                    swap32(g, u);
                    if (lane < 32 && (lane & 15) == 0 && row < st.nrows)
                        st.y[b * st.ldy + st.r0 + row] = silu_mul_h(g, u);
                } else {
                    if ((lane & 15) == 0 && row < st.nrows) st.y[b * st.ldy + st.r0 + row] = f2h_bits(v);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[b][r] = 0.f;
            }
        }
    }
    // no transfer into this workgroup's LDS may outlive it (a wave with no
    // stage issued dummy ones; every other transfer was waited for above)
    if (T == 0) wait_vmcnt<0>();
    if constexpr (SW) {
        lds_barrier();  // every wave's partials are in
        if (my_win == 0 && lane < 4 * NB) {
            const int b = lane >> 2, r = lane & 3;
            for (int t = 0; t < T; ++t) {
                const RowsStage st = stage_at(t);
                float v = 0.f;
                for (int w = 0; w < NW; ++w) {
                    uint32_t bits;
                    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                                 : "=v"(bits)
                                 : "v"(part0 + 4u * (((t * WV + wave + w) * NB + b) * 4 + r)));
                    v += __builtin_bit_cast(float, bits);
                }
                if (r < st.nrows) st.y[b * st.ldy + st.r0 + r] = f2h_bits(v);
            }
        }
    }
}

// ---- MFMA batched GEMV (batch 3..16) ---------------------------------------------
// With B >= 3 rows of x every weight feeds B dot products and the dot2 path is
// VALU-bound.  Here the weights are dequantized in registers to exactly the
// fp16 values the reference's dequant produces ((q - 8) and q are exact in
// packed fp16, the packed multiply by d rounds once) and enter
// v_mfma_f32_16x16x32_f16 as A = 16 rows x one 32-weight block; x of up to 16
// batch rows is B, permuted into the same element order.  Lane group g
// (lanes 16g..16g+15) covers qs dword g of each block: for Q4_0 the elements
// 4g..4g+3 (low nibbles) and 16+4g..19+4g (high nibbles), for Q8_0 the
// elements 8g..8g+7; the MFMA sum over k is order-free, so A and B only have
// to agree.
//
// Row tiles of 16*RT rows (RT = 1 or 2 MFMA tiles) are dealt to a resident
// grid of workgroups (tile blockIdx.x, then + gridDim.x, ...).  Within a tile
// the kMfmaWaves waves take the super-blocks of K in turn (wave w: w, w + 8,
// ...), so at any moment they read 8 adjacent super-blocks of the same rows.
// A stage is one wave's super-block of the tile's rows (RT*2304 B for Q4_0,
// RT*4352 B for Q8_0).  Each wave keeps kMfmaDepth stages and their x in
// flight in registers across tile boundaries (ordinary loads, so the compiler
// tracks every wait), copies the oldest into its LDS slot, where row r occupies
// bytes [r*SB, r*SB + SB), and feeds the MFMAs from there.  At the end of a
// tile the waves' partial tiles are summed through LDS in wave order (so the
// result does not depend on timing) behind an LDS-only barrier that leaves the
// next tile's loads in flight.

constexpr int kMfmaWaves = 8;  // waves per workgroup, interleaved over K
constexpr int kMfmaDepth = 2;  // stages in flight per wave

// LDS slot of one wave: the stage rounded up to whole 1 KB rows of 64 chunks,
// so every lane stores every chunk it holds without a bounds test.
template <Fmt F, int RT>
constexpr int mfma_slot_bytes() { return (16 * RT * Layout<F>::kSbChunks + 63) / 64 * 1024; }
// partial tiles of all waves: [wave][t][chain][v][lane] fp32
template <int RT>
constexpr int mfma_red_bytes() { return kMfmaWaves * RT * 2 * 4 * 64 * 4; }
template <Fmt F, int RT>
constexpr int mfma_lds_bytes() { return kMfmaWaves * mfma_slot_bytes<F, RT>() + 2 * mfma_red_bytes<RT>(); }

// Raw x of block `gb` for lane group g, kept in the register pairs the loads
// fill (regrouping them costs a copy of every pair).
struct XRaw {
    uint2 a, b;
};
template <Fmt F>
__device__ __forceinline__ XRaw load_x_b(const uint16_t* __restrict__ xb, int gb, int g) {
    if constexpr (F == Fmt::Q4_0) {
        // elements 4g..4g+3 and 16+4g..19+4g
        return {*reinterpret_cast<const uint2*>(xb + 32 * gb + 4 * g),
                *reinterpret_cast<const uint2*>(xb + 32 * gb + 16 + 4 * g)};
    } else {
        // elements 8g..8g+7
        const uint4 v = *reinterpret_cast<const uint4*>(xb + 32 * gb + 8 * g);
        return {make_uint2(v.x, v.y), make_uint2(v.z, v.w)};
    }
}

// B operand of a block from its raw x, in weight_a_operand's element order.
template <Fmt F>
__device__ __forceinline__ half8_t x_b_operand(const XRaw& r) {
    uint32_t p[4];
    if constexpr (F == Fmt::Q4_0) {
        // (x4g, x4g+2) (x16+4g, x18+4g) (x4g+1, x4g+3) (x17+4g, x19+4g)
        p[0] = __builtin_amdgcn_perm(r.a.y, r.a.x, kSelLo);
        p[1] = __builtin_amdgcn_perm(r.b.y, r.b.x, kSelLo);
        p[2] = __builtin_amdgcn_perm(r.a.y, r.a.x, kSelHi);
        p[3] = __builtin_amdgcn_perm(r.b.y, r.b.x, kSelHi);
    } else {
        // (x0, x2) (x1, x3) (x4, x6) (x5, x7) of elements 8g..8g+7
        p[0] = __builtin_amdgcn_perm(r.a.y, r.a.x, kSelLo);
        p[1] = __builtin_amdgcn_perm(r.a.y, r.a.x, kSelHi);
        p[2] = __builtin_amdgcn_perm(r.b.y, r.b.x, kSelLo);
        p[3] = __builtin_amdgcn_perm(r.b.y, r.b.x, kSelHi);
    }
    return __builtin_bit_cast(half8_t, make_uint4(p[0], p[1], p[2], p[3]));
}

// The dwords of a block pair (blocks 2P, 2P+1 of a stage row, 4-byte aligned)
// that lane group g needs: Q4_0 {d word of each block, qs dwords g and g+1 of
// the even block (unaligned by 2), qs dword g of the odd block}; Q8_0 {d words,
// qs dwords 2g..2g+2 of the even block, 2g and 2g+1 of the odd one}.
template <Fmt F>
struct PairWords {
    static constexpr int N = F == Fmt::Q4_0 ? 5 : 7;
    uint32_t w[N];
};
template <Fmt F>
__device__ __forceinline__ PairWords<F> pair_words(const uint32_t* pr, int g) {
    PairWords<F> p;
    if constexpr (F == Fmt::Q4_0) {
        p.w[0] = pr[0];
        p.w[1] = pr[4];
        p.w[2] = pr[g];
        p.w[3] = pr[g + 1];
        p.w[4] = pr[5 + g];
    } else {
        p.w[0] = pr[0];
        p.w[1] = pr[8];
        p.w[2] = pr[2 * g];
        p.w[3] = pr[2 * g + 1];
        p.w[4] = pr[2 * g + 2];
        p.w[5] = pr[9 + 2 * g];
        p.w[6] = pr[10 + 2 * g];
    }
    return p;
}

// A operand of block ODD of a pair for lane group g: bit-exact fp16 weights in
// x_b_operand's order.
template <Fmt F, int ODD>
__device__ __forceinline__ half8_t weight_a_operand(const PairWords<F>& p, const NibUnpack& nu) {
    uint32_t dbits;
    half2_t h[4];
    if constexpr (F == Fmt::Q4_0) {
        uint32_t q;
        if constexpr (ODD == 0) {
            dbits = p.w[0] & 0xFFFFu;
            q = align2(p.w[2], p.w[3]);
        } else {
            dbits = p.w[1] >> 16;
            q = p.w[4];
        }
        const half2_t lo_off = {static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f)};
        const half2_t hi_off = {static_cast<half_t>(-72.0f), static_cast<half_t>(-72.0f)};
        const uint32_t qs = q >> 8;
        h[0] = __builtin_bit_cast(half2_t, nu.lo_c(q)) + lo_off;
        h[1] = __builtin_bit_cast(half2_t, nu.hi_c(q)) + hi_off;
        h[2] = __builtin_bit_cast(half2_t, nu.lo_c(qs)) + lo_off;
        h[3] = __builtin_bit_cast(half2_t, nu.hi_c(qs)) + hi_off;
    } else {
        uint32_t q0, q1;
        if constexpr (ODD == 0) {
            dbits = p.w[0] & 0xFFFFu;
            q0 = align2(p.w[2], p.w[3]);
            q1 = align2(p.w[3], p.w[4]);
        } else {
            dbits = p.w[1] >> 16;
            q0 = p.w[5];
            q1 = p.w[6];
        }
        const half2_t off = {static_cast<half_t>(-1152.0f), static_cast<half_t>(-1152.0f)};
        const uint32_t u0 = q0 ^ 0x80808080u, u1 = q1 ^ 0x80808080u;
        h[0] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u0, 0x04020400u)) + off;
        h[1] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u0, 0x04030401u)) + off;
        h[2] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u1, 0x04020400u)) + off;
        h[3] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u1, 0x04030401u)) + off;
    }
    const half_t d = __builtin_bit_cast(half_t, static_cast<uint16_t>(dbits));
    const half2_t dd = {d, d};
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __builtin_bit_cast(uint32_t, h[i] * dd);
    return __builtin_bit_cast(half8_t, make_uint4(w[0], w[1], w[2], w[3]));
}

// acc += the 8 blocks of one super-block row tile (A from the pair words, B
// from xb), one block at a time: the scheduling barrier after each MFMA keeps
// the compiler from building all eight operands first, which would cost the
// registers that hold the stages in flight.
template <Fmt F, int J>
__device__ __forceinline__ void mfma_block(float4_t (&acc)[2], const PairWords<F> (&pw)[4], const NibUnpack& nu,
                                           const half8_t (&xb)[4]) {
    acc[J % 2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(weight_a_operand<F, J % 2>(pw[J / 2], nu), xb[J / 2],
                                                        acc[J % 2], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
}
template <Fmt F, int... J>
__device__ __forceinline__ void mfma_superblock(float4_t (&acc)[2], const PairWords<F> (&pw)[4], const NibUnpack& nu,
                                                const half8_t (&xb)[4], std::integer_sequence<int, J...>) {
    (mfma_block<F, J>(acc, pw, nu, xb), ...);
}

template <Fmt F, int RT>
__global__ __launch_bounds__(kMfmaWaves * 64) void gguf_gemv_mfma(const uint8_t* __restrict__ W,
                                                                  const uint16_t* __restrict__ X,
                                                                  uint16_t* __restrict__ Y, int M, int K, int nb,
                                                                  int64_t ldx, int64_t ldy) {
    using L = Layout<F>;
    constexpr int kRows = 16 * RT;
    constexpr int kChunks = kRows * L::kSbChunks;  // 16-byte chunks of a stage
    constexpr int CPL = (kChunks + 63) / 64;
    constexpr int kRowDw = L::kSbBytes / 4;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    uint8_t* stage = smem + wave * mfma_slot_bytes<F, RT>();
    float* red0 = reinterpret_cast<float*>(smem + kMfmaWaves * mfma_slot_bytes<F, RT>());
    const int S = K >> 8;  // super-blocks per row
    const int64_t row_bytes = static_cast<int64_t>(S) * L::kSbBytes;
    const int ntiles = (M + kRows - 1) / kRows;
    const int T = (ntiles - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
    const int nst = S > wave ? (S - 1 - wave) / kMfmaWaves + 1 : 0;  // stages of this wave per tile
    const NibUnpack nu;
    const int g = lane >> 4, bcol = lane & 15;

    // With nb <= 8 one B operand carries two blocks: columns 0-7 hold tokens
    // 0-7 of block 2i, columns 8-15 the same tokens of block 2i+1.  Even blocks
    // accumulate into chain 0, whose valid columns are 0-7, odd blocks into
    // chain 1, valid in columns 8-15; the other half of each chain is never read.
    // Lanes of tokens past nb read x row 0; lanes of chunks past the stage or
    // past row M read the stage's first chunk.  Every load is valid and
    // unconditional (a load under a branch makes the compiler wait for all
    // loads in flight), and what the extra lanes bring only reaches MFMA
    // columns and rows that are never read: an MFMA row depends on its A row
    // only, a column on its B column only, so LDS rows past M (duplicate
    // bytes, scale possibly Inf/NaN) and columns past nb stay apart.
    const int tok = bcol & 7, half = bcol >> 3;
    const uint16_t* xrow = X + (tok < nb ? tok : 0) * ldx;
    // chunk j of this lane: stage row c / kSbChunks, chunk c % kSbChunks of it
    int crow[CPL];
    uint32_t coff[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = 64 * j + lane;
        crow[j] = c < kChunks ? c / L::kSbChunks : 0;
        coff[j] = c < kChunks ? 16 * (c - crow[j] * L::kSbChunks) : 0u;
    }

    uint4 pre[kMfmaDepth][CPL];
    XRaw xr[kMfmaDepth][4];
    float4_t acc[RT][2];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t][0] = acc[t][1] = float4_t{0.f, 0.f, 0.f, 0.f};

    // next stage to load: tile lk of this workgroup, stage li of this wave;
    // past the last one the last stage is loaded again (never computed)
    int lk = 0, li = 0;
    auto load = [&](auto slot) {
        constexpr int sl = decltype(slot)::value;
        const bool past = lk >= T;
        const int r0 = kRows * (static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) * (past ? T - 1 : lk));
        const int sb = wave + kMfmaWaves * (past ? nst - 1 : li);
        const int nrows = min(kRows, M - r0);
        const uint8_t* src = W + static_cast<int64_t>(r0) * row_bytes + static_cast<int64_t>(sb) * L::kSbBytes;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t off = crow[j] < nrows ? crow[j] * row_bytes + coff[j] : 0;
            pre[sl][j] = load_nt16(src + off);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[sl][i] = load_x_b<F>(xrow, 8 * sb + 2 * i + half, g);
        if (++li == nst) {
            li = 0;
            ++lk;
        }
    };
    // End of tile ck: sum the waves' partial tiles in wave order and store the
    // rows (one output per thread).  red alternates between two buffers: the
    // barrier of the next tile separates this tile's reads of one buffer from
    // its next writes.
    int ck = 0;
    auto finish_tile = [&]() {
        float* red = red0 + (ck & 1) * (mfma_red_bytes<RT>() / 4);
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
#pragma unroll
                for (int v = 0; v < 4; ++v) red[(((wave * RT + t) * 2 + c) * 4 + v) * 64 + lane] = acc[t][c][v];
                acc[t][c] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
        lds_barrier();
        const int r0 = kRows * (static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) * ck);
        const int r = static_cast<int>(threadIdx.x) / nb, b = static_cast<int>(threadIdx.x) - r * nb;
        if (r < min(kRows, M - r0)) {
            const int t = r >> 4, r16 = r & 15;
            const int src_lane = 16 * (r16 >> 2) + b, v = r16 & 3;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < kMfmaWaves; ++w)
                sum += red[(((w * RT + t) * 2 + 0) * 4 + v) * 64 + src_lane] +
                       red[(((w * RT + t) * 2 + 1) * 4 + v) * 64 + src_lane + 8];
            Y[b * ldy + r0 + r] = f2h_bits(sum);
        }
        ++ck;
    };
    // next stage to compute: stage ci of the current tile
    int ci = 0;
    auto compute = [&](auto slot) {
        constexpr int sl = decltype(slot)::value;
#pragma unroll
        for (int j = 0; j < CPL; ++j) *reinterpret_cast<uint4*>(stage + 16 * (64 * j + lane)) = pre[sl][j];
        wave_lds_sync();
        half8_t xb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xb[i] = x_b_operand<F>(xr[sl][i]);
        // every LDS word of the stage this lane needs, read before any is used,
        // so the stage waits for LDS once
        PairWords<F> pw[RT][4];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t* row = reinterpret_cast<const uint32_t*>(stage) + (16 * t + bcol) * kRowDw;
#pragma unroll
            for (int P = 0; P < 4; ++P) pw[t][P] = pair_words<F>(row + P * (Layout<F>::kBlockBytes / 2), g);
        }
#pragma unroll
        for (int t = 0; t < RT; ++t) mfma_superblock<F>(acc[t], pw[t], nu, xb, std::make_integer_sequence<int, 8>{});
        if (++ci == nst) {
            ci = 0;
            finish_tile();
        }
    };
    static_assert(kRows * 8 <= kMfmaWaves * 64, "one output per thread per tile");

    if (nst == 0) {
        // K has fewer super-blocks than the workgroup has waves: this wave
        // adds zero partials to every tile's sum
        for (int k = 0; k < T; ++k) finish_tile();
        return;
    }
    const int Q = T * nst;  // stages of this wave in all its tiles
    // slots cycle 0 .. kMfmaDepth-1; the steady loop issues every load
    // unconditionally and the tail only computes
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    static_assert(kMfmaDepth == 2 || kMfmaDepth == 3, "two or three slots");
    load(I0{});
    load(I1{});
    if constexpr (kMfmaDepth == 3) load(I2{});
    int q = 0;
    for (; q + kMfmaDepth < Q; q += kMfmaDepth) {
        compute(I0{});
        load(I0{});
        compute(I1{});
        load(I1{});
        if constexpr (kMfmaDepth == 3) {
            compute(I2{});
            load(I2{});
        }
    }
    if (q < Q) compute(I0{});
    if (q + 1 < Q) compute(I1{});
    if constexpr (kMfmaDepth == 3)
        if (q + 2 < Q) compute(I2{});
}

// ---- Q4_0 batched GEMV, batch 3..8: raw codes on the matrix cores ------------
// The weights enter v_mfma_f32_16x16x32_f16 as their exponent-trick codes, not
// dequantized: 1024 + q for low nibbles, 64 + q for high nibbles, one
// v_and_or_b32 per pair of weights.  Per block b and batch row t the MFMA then
// yields S = sum_k x_k * code_k, and
//     sum_k x_k * (q_k - 8) = S - c,   c = 1032 * sum_lo x + 72 * sum_hi x,
// exactly as in the batch-1 path; the block's scale multiplies (S - c) in
// fp32 afterwards (v_fma_mix, one per output).  c itself comes from one more
// MFMA per block pair, x times a constant operand (-1032 / -72), and enters
// the weight MFMAs as their C input, so no VALU work computes it.
//
// Operands: A = x, 16 slots = batch rows 0-7 of block 2p (slots 0-7) and of
// block 2p+1 (slots 8-15); B = weights, 16 columns = rows 0-7 of a row group
// with block 2p (columns 0-7) and block 2p+1 (columns 8-15).  Lane group g
// (lanes 16g..16g+15) holds k-group g of every operand: elements 4g..4g+3
// (low nibbles of qs dword g) and 16+4g..19+4g (its high nibbles), so x is read
// from LDS in its natural order (two 8-byte reads) and only the outputs whose
// slot and column take the same block are valid: lanes 0-7 and 16-23 (block
// 2p, batch rows 4g+v) and lanes 40-47 and 56-63 (block 2p+1).  Each lane
// holds one column, i.e. one (row, block), so it applies a single scale.
//
// Work split: a workgroup of 8 waves owns a tile of RT rows (32 or 16) at a
// time; wave w takes super-blocks w, w+8, ... of K.  A stage is the tile's rows
// x one super-block (RT*144 bytes of weights) plus x of its 256 columns for 8
// batch rows (4 KiB), moved by LDS DMA; every wave keeps two stages in flight.
// At the end of a tile the waves' partial sums meet in LDS and are added in
// wave order, so results do not depend on timing.
// Weight operand of one block pair from its two permuted qs dwords: the
// exponent-trick codes (1024 + q low nibbles, 64 + q high nibbles), or with
// kCodesExact the exact q - 8 (the codes plus kneg = -1032 / -72, four packed
// fp16 adds).
__device__ __forceinline__ half8_t codes_operand(uint32_t p01, uint32_t p23, const NibUnpack& nu, half8_t kneg) {
    const half8_t c = __builtin_bit_cast(half8_t, make_uint4(nu.lo_c(p01), nu.lo_c(p23), nu.hi_c(p01), nu.hi_c(p23)));
    if constexpr (kCodesExact) return c + kneg;
    return c;
}

namespace bq {
constexpr int kWaves = 8;
constexpr int kXStride = 1088;                  // LDS bytes per x transfer (2 batch rows + bank padding)
constexpr int kXBytes = 4 * kXStride;
template <int RT>
constexpr int w_dma() { return (RT * 9 + 63) / 64; }  // weight transfers per stage: 5 (RT 32), 3 (RT 16)
template <int RT>
constexpr int w_last_lanes() { return RT * 9 - 64 * (w_dma<RT>() - 1); }
template <int RT>
constexpr int slot_bytes() { return RT * 144 + kXBytes; }
template <int RT>
constexpr int red_bytes() { return kWaves * 8 * RT * 4; }
template <int RT>
constexpr int lds_bytes() { return kWaves * 2 * slot_bytes<RT>() + 2 * red_bytes<RT>(); }
}  // namespace bq

template <int RT, int XT>
__global__ __launch_bounds__(bq::kWaves * 64) void gguf_gemv_q4_codes(const uint8_t* __restrict__ W,
                                                                     const uint16_t* __restrict__ X,
                                                                     uint16_t* __restrict__ Y, int M, int K, int nb,
                                                                     int64_t ldx, int64_t ldy) {
    constexpr int NRG = RT / 8;        // row groups of 8 per stage
    constexpr int NWD = bq::w_dma<RT>();
    // x transfers per stage: 4 (batch rows 0-7), or 2 where batch <= 4
    static_assert(XT == 2 || XT == 4, "x transfers per stage");
    constexpr int kOps = NWD + XT;     // transfers per stage
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int S = K >> 8;
    const uint32_t row_bytes = static_cast<uint32_t>(S) * 144u;
    const int ntiles = (M + RT - 1) / RT;
    const int T = (ntiles - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
    const int nst = S > wave ? (S - 1 - wave) / bq::kWaves + 1 : 0;  // stages of this wave per tile
    const int Q = T * nst;
    const uint32_t lds0 = lds_addr(lds);
    const uint32_t slot0 = lds0 + wave * 2 * bq::slot_bytes<RT>();
    float* red0 = reinterpret_cast<float*>(lds + bq::kWaves * 2 * bq::slot_bytes<RT>());

    // transfer offsets.  x transfer j: batch rows 2j + (lane >> 5) (rows past
    // nb read row nb - 1), 16-byte chunk lane & 31 of the stage's 256 columns.
    uint32_t xoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = min(2 * j + (lane >> 5), nb - 1);
        xoff[j] = static_cast<uint32_t>(2 * (t * ldx + 8 * (lane & 31)));
    }
    // weight transfer j: chunk c = 64j + lane = row c / 9, chunk c % 9 of the
    // row's super-block (rows past the tile's last valid row read that row)
    auto w_offsets = [&](int nrows, uint32_t (&off)[NWD]) {
#pragma unroll
        for (int j = 0; j < NWD; ++j) {
            const int c = min(64 * j + lane, RT * 9 - 1);
            const int r = c / 9;
            off[j] = static_cast<uint32_t>(min(r, nrows - 1)) * row_bytes + 16u * static_cast<uint32_t>(c - 9 * r);
        }
    };
    uint32_t woff_full[NWD];
    w_offsets(RT, woff_full);

    // next stage to issue: tile ii of this workgroup, step ss of this wave
    int ii = 0, ss = 0;
    auto issue = [&](int q) {
        const uint32_t slot = slot0 + (q & 1) * bq::slot_bytes<RT>();
        const int sb = wave + bq::kWaves * ss;
        const int row0 = RT * (static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) * ii);
        const uint16_t* xb = X + 256 * sb;
#pragma unroll
        for (int j = 0; j < XT; ++j) dma16_asm(xoff[j], xb, slot + RT * 144 + bq::kXStride * j);
        const uint8_t* wb = W + static_cast<int64_t>(row0) * row_bytes + 144 * sb;
        uint32_t woff[NWD];
        const int nrows = min(RT, M - row0);
        if (nrows == RT) {
#pragma unroll
            for (int j = 0; j < NWD; ++j) woff[j] = woff_full[j];
        } else {
            w_offsets(nrows, woff);
        }
#pragma unroll
        for (int j = 0; j < NWD - 1; ++j) dma16_asm(woff[j], wb, slot + 1024 * j);
        if (lane < bq::w_last_lanes<RT>()) dma16_asm(woff[NWD - 1], wb, slot + 1024 * (NWD - 1));
        if (++ss == nst) {
            ss = 0;
            ++ii;
        }
    };

    // per-lane operand geometry
    const int g = lane >> 4, j = lane & 15, par = j >> 3;
    // x: batch row j & 7 of block 2p + par, elements 4g.. and 16+4g.. (bytes +32)
    // (batch rows past nb read row nb - 1, which the transfers hold)
    const int xt = min(j & 7, nb - 1);
    const uint32_t xrd = xt / 2 * bq::kXStride + (xt & 1) * 512 + 64 * par + 8 * g;
    // weights: row 8rg + (j & 7), block 2p + par; qs dword g starts at byte
    // 144r + 18(2p + par) + 2 + 4g, which is 2 mod 4 for the even block
    const uint32_t wrd = 144 * (j & 7) + (par ? 20 : 0) + 4 * g;
    const uint32_t drd = 144 * (j & 7) + 18 * par;
    const uint32_t sel01 = par ? 0x0C010C00u : 0x0C030C02u;
    const uint32_t sel23 = par ? 0x0C030C02u : 0x0C050C04u;
    const NibUnpack nu;
    const half8_t kneg = {static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f),
                          static_cast<half_t>(-1032.0f), static_cast<half_t>(-72.0f),   static_cast<half_t>(-72.0f),
                          static_cast<half_t>(-72.0f),   static_cast<half_t>(-72.0f)};

    float4_t acc[NRG];
#pragma unroll
    for (int r = 0; r < NRG; ++r) acc[r] = float4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int q) {
        const uint8_t* slot = lds + (slot0 - lds0) + (q & 1) * bq::slot_bytes<RT>();
        const uint8_t* xs = slot + RT * 144 + xrd;
        half8_t xa[4];
        float4_t dc[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint2 lo = *reinterpret_cast<const uint2*>(xs + 128 * p);
            const uint2 hi = *reinterpret_cast<const uint2*>(xs + 128 * p + 32);
            xa[p] = __builtin_bit_cast(half8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
            dc[p] = kCodesExact ? float4_t{0.f, 0.f, 0.f, 0.f}
                                : __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[p], kneg, float4_t{0.f, 0.f, 0.f, 0.f}, 0,
                                                                         0, 0);
        }
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint8_t* wr = slot + 1152 * rg + 36 * p;
                const uint32_t d0 = *reinterpret_cast<const uint32_t*>(wr + wrd);
                const uint32_t d1 = *reinterpret_cast<const uint32_t*>(wr + wrd + 4);
                const half_t dv = __builtin_bit_cast(half_t, *reinterpret_cast<const uint16_t*>(wr + drd));
                const uint32_t p01 = __builtin_amdgcn_perm(d1, d0, sel01);
                const uint32_t p23 = __builtin_amdgcn_perm(d1, d0, sel23);
                const half8_t wb = codes_operand(p01, p23, nu, kneg);
                const float4_t D = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[p], wb, dc[p], 0, 0, 0);
                const float dsc = static_cast<float>(dv);
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[rg][v] = __builtin_fmaf(dsc, D[v], acc[rg][v]);
            }
    };

    // End of tile ck: lanes 0-7 / 16-23 add the block-2p+1 partials of lanes
    // +40, write batch rows 4g+v of row 8rg + j to LDS; after the barrier each
    // of the first 8*RT threads sums one (batch row, row) over the waves.
    int ck = 0;
    auto finish_tile = [&]() {
        float* red = red0 + (ck & 1) * (bq::red_bytes<RT>() / 4);
        const int src = lane + 40 < 64 ? lane + 40 : lane;
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float o = __shfl(acc[rg][v], src, 64);
                if (g < 2 && j < 8) red[(wave * 8 + 4 * g + v) * RT + 8 * rg + j] = acc[rg][v] + o;
            }
            acc[rg] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
        lds_barrier();
        const int i = threadIdx.x;
        const int row0 = RT * (static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) * ck);
        if (i < 8 * RT) {
            const int t = i / RT, r = i - t * RT;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < bq::kWaves; ++w) sum += red[(w * 8 + t) * RT + r];
            if (t < nb && row0 + r < M) Y[t * ldy + row0 + r] = f2h_bits(sum);
        }
        ++ck;
    };

    if (nst == 0) {
        // K has fewer super-blocks than the workgroup has waves: this wave
        // adds zero partials to every tile's sum
        for (int k = 0; k < T; ++k) finish_tile();
        return;
    }
    issue(0);
    if (Q > 1) issue(1);
    int cs = 0;  // step of the stage being computed within its tile
    for (int q = 0; q < Q; ++q) {
        if (q + 1 < Q)
            wait_vmcnt_asm<kOps>();  // stage q has landed (stage q+1 may be in flight)
        else
            wait_vmcnt_asm<0>();
        compute(q);
        // every LDS read of this slot has returned before the DMA refills it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (q + 2 < Q) issue(q + 2);
        if (++cs == nst) {
            cs = 0;
            finish_tile();
        }
    }
}

template <int RT, int XT>
int launch_q4_codes(const void* w, const uint16_t* x, uint16_t* y, int M, int K, int64_t batch, int64_t ldx,
                    int64_t ldy, hipStream_t stream) {
    constexpr size_t lds = bq::lds_bytes<RT>();
    const void* fn = reinterpret_cast<const void*>(&gguf_gemv_q4_codes<RT, XT>);
    if (int rc = prepare_lds(fn, lds)) return rc;
    const int tiles = (M + RT - 1) / RT;
    const int resident = blocks_per_cu(fn, lds, bq::kWaves * 64) * cu_count();
    const int grid = std::min(tiles, resident);
    hipLaunchKernelGGL((gguf_gemv_q4_codes<RT, XT>), dim3(grid), dim3(bq::kWaves * 64), lds, stream,
                       static_cast<const uint8_t*>(w), x, y, M, K, static_cast<int>(batch), ldx, ldy);
    return check_hip(hipGetLastError(), "gguf_gemv_q4_codes launch");
}

// ---- Q4_0 codes on MFMA with x held in registers (in_dim <= 8192) ----------
//
// Same operands and arithmetic as gguf_gemv_q4_codes, different data
// movement.  Wave w of a 16-wave workgroup always takes super-blocks w and
// w+16 of K, for every 16-row tile the workgroup owns, so its slice of x (up
// to 2 super-blocks x 8 batch rows, 8 KiB) is loaded once instead of once per
// tile.  LDS then holds weights only: 4 stage slots per wave, so a tile's
// whole K is in flight at once.  The x slice comes in by LDS DMA (2 batch rows
// x 512 contiguous bytes per transfer) into the wave's slots and is read into
// registers before the first weights are issued; register loads straight
// from HBM gathered 8 batch rows per instruction and took ~4 us longer per
// launch.
namespace bx {
constexpr int kRT = 16;  // rows per tile
constexpr int kNWD = (kRT * 9 + 63) / 64;                  // weight transfers per stage (3)
constexpr int kLastLanes = kRT * 9 - 64 * (kNWD - 1);      // lanes of the last one (16)
constexpr int kSlotBytes = kRT * 144;                      // one super-block of the tile's rows
// WV waves per workgroup, at most NSB super-blocks of K per wave, NS stage
// slots per wave.
template <int WV, int NSB, int NS>
struct Cfg {
    static constexpr int kWaves = WV, kNSB = NSB, kNS = NS;
    static constexpr int kRedBytes = WV * 8 * kRT * 4;  // one tile's partial sums
    static constexpr int kLdsBytes = WV * NS * kSlotBytes + 2 * kRedBytes;
    static_assert(NS * kSlotBytes >= NSB * 4096, "the x slice is staged in the wave's slots");
    static_assert(kLdsBytes <= 160 * 1024, "LDS of one compute unit");
};
// 16 waves x 2 super-blocks (in_dim <= 8192), 4 slots: a 16-row tile's whole
// K in flight at once.  The offset corrections are recomputed per stage (4
// MFMAs) to stay within the 128 registers of a 1024-thread workgroup.
// Measured against 8 waves x 4 super-blocks with 8 slots and the corrections
// kept in registers (batch 8, us): 28672x8192 31.7 / 34.3, 13003x4096
// 13.7 / 15.8, 9000x5120 12.2 / 14.2.
using Tall = Cfg<16, 2, 4>;
// in_dim <= 4096: 8 waves x 2 super-blocks, 4 slots (80 KiB, two workgroups
// per CU, each with its own barrier) where there are at least two 16-row
// tiles per CU.  Batch 3 / 4 / 8 against Tall, us: 11008x4096 9.5 / 9.6 /
// 10.1 against 11.0 / 11.1 / 11.7; 13003x4096 12.0 / 12.2 / 12.9 against
// 13.9 / 13.9 / 14.4; the 7B q/k/v group 10.0 / 10.3 / 10.8 against 11.6 /
// 11.8 / 12.2 and gate/up pair 17.4 / 17.5 / 18.0 against 19.9 / 20.0 /
// 20.4; with one tile per CU (4096x4096 at batch 3) 5.45 against 5.17.
using Half = Cfg<8, 2, 4>;

// Where a launch reads weights and writes results.  MODE 0: one matrix
// (w[0], y[0], m[0]); 1: up to 4 matrices of the same in_dim sharing x, whose
// 16-row tiles are numbered one matrix after another (tile_end[i]: one past
// matrix i's last tile; the entries past the last matrix repeat the total);
// 2: gate/up pairs, w[0] = gate and w[1] = up with m[0] rows each: tile t
// holds gate rows 8t..8t+7 (row group 0) and the same up rows (row group 1),
// and y[0][b*ldy[0] + r] receives h = fp16(silu(fp16 gate) * fp16 up).
// tile_end[kMaxGroup - 1] is the launch's tile count in every mode.
struct Target {
    const uint8_t* w[kMaxGroup];
    uint16_t* y[kMaxGroup];
    int64_t ldy[kMaxGroup];
    int m[kMaxGroup];
    int tile_end[kMaxGroup];
};

// One tile: the weights of its first row (pairing: gate and up), where its
// results go, its first row and its matrix's row count.
struct Tile {
    const uint8_t *w0, *w1;
    uint16_t* y;
    int64_t ldy;
    int row0, m;
};
template <int MODE>
__device__ __forceinline__ Tile tile_of(const Target& tg, int t) {
    Tile r;
    if constexpr (MODE == 1) {
        const int i = (t >= tg.tile_end[0]) + (t >= tg.tile_end[1]) + (t >= tg.tile_end[2]);
        int first;
        switch (i) {
            case 0: r.w0 = tg.w[0], r.y = tg.y[0], r.ldy = tg.ldy[0], r.m = tg.m[0], first = 0; break;
            case 1: r.w0 = tg.w[1], r.y = tg.y[1], r.ldy = tg.ldy[1], r.m = tg.m[1], first = tg.tile_end[0]; break;
            case 2: r.w0 = tg.w[2], r.y = tg.y[2], r.ldy = tg.ldy[2], r.m = tg.m[2], first = tg.tile_end[1]; break;
            default: r.w0 = tg.w[3], r.y = tg.y[3], r.ldy = tg.ldy[3], r.m = tg.m[3], first = tg.tile_end[2]; break;
        }
        r.w1 = r.w0;
        r.row0 = kRT * (t - first);
    } else {
        r.w0 = tg.w[0], r.w1 = tg.w[MODE == 2 ? 1 : 0], r.y = tg.y[0], r.ldy = tg.ldy[0], r.m = tg.m[0];
        r.row0 = (MODE == 2 ? kRT / 2 : kRT) * t;
    }
    return r;
}
}  // namespace bx

template <class C, int MODE>
__global__ __launch_bounds__(C::kWaves * 64) void gguf_gemv_q4_xreg(const bx::Target tg,
                                                                    const uint16_t* __restrict__ X, int K, int nb,
                                                                    int64_t ldx) {
    constexpr int RT = bx::kRT, NRG = RT / 8, NS = C::kNS;
    // transfers per stage: 3 (16 rows of one matrix); pairing: 2 per matrix
    // (chunks 0-63 of the 8 rows, then chunks 64-71 on 8 lanes)
    constexpr int NWD = MODE == 2 ? 4 : bx::kNWD;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int S = K >> 8;
    const uint32_t row_bytes = static_cast<uint32_t>(S) * 144u;
    const int ntiles = tg.tile_end[kMaxGroup - 1];
    const int T = (ntiles - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
    const int nst = S > wave ? (S - 1 - wave) / C::kWaves + 1 : 0;  // super-blocks of this wave (<= NSB)
    const int Q = T * nst;
    const uint32_t lds0 = lds_addr(lds);
    const uint32_t slot0 = lds0 + wave * NS * bx::kSlotBytes;
    float* red0 = reinterpret_cast<float*>(lds + C::kWaves * NS * bx::kSlotBytes);

    // weight transfer j: chunk c = 64j + lane = row c / 9, chunk c % 9 of the
    // row's super-block (rows past the tile's last valid row read that row).
    // Pairing: chunks of one matrix's 8 rows, c = lane, then c = 64 + lane.
    constexpr int NOFF = MODE == 2 ? 2 : NWD;
    constexpr int kChunks = MODE == 2 ? 72 : RT * 9;
    auto w_offsets = [&](int nrows, uint32_t (&off)[NOFF]) {
#pragma unroll
        for (int j = 0; j < NOFF; ++j) {
            const int c = min(64 * j + lane, kChunks - 1);
            const int r = c / 9;
            off[j] = static_cast<uint32_t>(min(r, nrows - 1)) * row_bytes + 16u * static_cast<uint32_t>(c - 9 * r);
        }
    };
    uint32_t woff_full[NOFF];
    w_offsets(MODE == 2 ? RT / 2 : RT, woff_full);

    int ii = 0, ss = 0, qs = 0;  // next stage to issue: tile ii, super-block step ss, slot qs
    auto issue = [&]() {
        const uint32_t slot = slot0 + qs * bx::kSlotBytes;
        const int sb = wave + C::kWaves * ss;
        const bx::Tile tl = bx::tile_of<MODE>(tg, static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) * ii);
        const int64_t at = static_cast<int64_t>(tl.row0) * row_bytes + 144 * sb;
        uint32_t woff[NOFF];
        const int nrows = min(MODE == 2 ? RT / 2 : RT, tl.m - tl.row0);
        if (nrows == (MODE == 2 ? RT / 2 : RT)) {
#pragma unroll
            for (int j = 0; j < NOFF; ++j) woff[j] = woff_full[j];
        } else {
            w_offsets(nrows, woff);
        }
        if constexpr (MODE == 2) {
            // gate rows into row group 0, up rows into row group 1
            dma16_asm(woff[0], tl.w0 + at, slot);
            if (lane < 8) dma16_asm(woff[1], tl.w0 + at, slot + 1024);
            dma16_asm(woff[0], tl.w1 + at, slot + 1152);
            if (lane < 8) dma16_asm(woff[1], tl.w1 + at, slot + 1152 + 1024);
        } else {
            const uint8_t* wb = tl.w0 + at;
#pragma unroll
            for (int j = 0; j < NWD - 1; ++j) dma16_asm(woff[j], wb, slot + 1024 * j);
            if (lane < bx::kLastLanes) dma16_asm(woff[NWD - 1], wb, slot + 1024 * (NWD - 1));
        }
        if (++ss == nst) {
            ss = 0;
            ++ii;
        }
        if (++qs == NS) qs = 0;
    };

    // per-lane operand geometry, as in gguf_gemv_q4_codes
    const int g = lane >> 4, j = lane & 15, par = j >> 3;
    const uint32_t wrd = 144 * (j & 7) + (par ? 20 : 0) + 4 * g;
    const uint32_t drd = 144 * (j & 7) + 18 * par;
    const uint32_t sel01 = par ? 0x0C010C00u : 0x0C030C02u;
    const uint32_t sel23 = par ? 0x0C030C02u : 0x0C050C04u;
    const NibUnpack nu;

    int ck = 0;
    float4_t acc[NRG];
#pragma unroll
    for (int r = 0; r < NRG; ++r) acc[r] = float4_t{0.f, 0.f, 0.f, 0.f};
    auto finish_tile = [&]() {
        float* red = red0 + (ck & 1) * (C::kRedBytes / 4);
        const int src = lane + 40 < 64 ? lane + 40 : lane;
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float o = __shfl(acc[rg][v], src, 64);
                if (g < 2 && j < 8) red[(wave * 8 + 4 * g + v) * RT + 8 * rg + j] = acc[rg][v] + o;
            }
            acc[rg] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
        lds_barrier();
        const int i = threadIdx.x;
        const bx::Tile tl = bx::tile_of<MODE>(tg, static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) * ck);
        if constexpr (MODE == 2) {
            // one thread per (batch row, pair): gate in rows 0-7, up in rows 8-15
            if (i < 4 * RT) {
                const int t = i >> 3, r = i & 7;
                float gs = 0.f, us = 0.f;
#pragma unroll
                for (int w = 0; w < C::kWaves; ++w) {
                    gs += red[(w * 8 + t) * RT + r];
                    us += red[(w * 8 + t) * RT + 8 + r];
                }
                if (t < nb && tl.row0 + r < tl.m) tl.y[t * tl.ldy + tl.row0 + r] = silu_mul_h(gs, us);
            }
        } else if (i < 8 * RT) {
            const int t = i / RT, r = i - t * RT;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < C::kWaves; ++w) sum += red[(w * 8 + t) * RT + r];
            if (t < nb && tl.row0 + r < tl.m) tl.y[t * tl.ldy + tl.row0 + r] = f2h_bits(sum);
        }
        ++ck;
    };

    if (nst == 0) {
        // K has fewer super-blocks than the workgroup has waves: this wave
        // adds zero partials to every tile's sum
        for (int k = 0; k < T; ++k) finish_tile();
        return;
    }

    // x slice: 4 transfers per super-block into the wave's slots (transfer jj
    // holds batch rows 2jj, 2jj+1, rows past nb repeat row nb - 1; 2 where
    // nb <= 4; the super-blocks past this wave's last repeat it), then into
    // registers.
    half8_t xa[C::kNSB][4];
    {
        const int nxt = nb <= 4 ? 2 : 4;
#pragma unroll
        for (int s2 = 0; s2 < C::kNSB; ++s2) {
            const int sb = wave + C::kWaves * min(s2, nst - 1);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                if (jj >= nxt) break;
                const int tr = min(2 * jj + (lane >> 5), nb - 1);
                dma16_asm(static_cast<uint32_t>(2 * (tr * ldx + 8 * (lane & 31))), X + 256 * sb,
                          slot0 + 4096 * s2 + 1024 * jj);
            }
        }
        wait_vmcnt_asm<0>();
        // lane (g, j): batch row j & 7 of block 2p + par, elements 4g.. and 16+4g..
        const int t = min(j & 7, nb - 1);
        const uint8_t* xl = lds + (slot0 - lds0) + (t >> 1) * 1024 + (t & 1) * 512 + 2 * (32 * par + 4 * g);
#pragma unroll
        for (int s2 = 0; s2 < C::kNSB; ++s2)
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint2 lo = *reinterpret_cast<const uint2*>(xl + 4096 * s2 + 128 * p);
                const uint2 hi = *reinterpret_cast<const uint2*>(xl + 4096 * s2 + 128 * p + 32);
                xa[s2][p] = __builtin_bit_cast(half8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
            }
        // the reads have returned before transfers overwrite the slots
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    int issued = min(Q, NS);  // stages of weights issued
    for (int q = 0; q < issued; ++q) issue();

    const half8_t kneg = {static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f),
                          static_cast<half_t>(-1032.0f), static_cast<half_t>(-72.0f),   static_cast<half_t>(-72.0f),
                          static_cast<half_t>(-72.0f),   static_cast<half_t>(-72.0f)};
    float4_t dc[4];  // offset corrections of the stage's 4 block pairs

    int q = 0, cslot = 0;
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int s2 = 0; s2 < C::kNSB; ++s2) {
            if (s2 < nst) {
                // stages of weights issued after stage q
                switch (issued - 1 - q) {
                    case 0: wait_vmcnt_asm<0>(); break;
                    case 1: wait_vmcnt_asm<1 * NWD>(); break;
                    case 2: wait_vmcnt_asm<2 * NWD>(); break;
                    case 3: wait_vmcnt_asm<3 * NWD>(); break;
                    case 4: wait_vmcnt_asm<4 * NWD>(); break;
                    case 5: wait_vmcnt_asm<5 * NWD>(); break;
                    case 6: wait_vmcnt_asm<6 * NWD>(); break;
                    default: wait_vmcnt_asm<(NS - 1) * NWD>(); break;
                }
                const uint8_t* sl = lds + (slot0 - lds0) + cslot * bx::kSlotBytes;
#pragma unroll
                for (int p = 0; p < 4; ++p)
                    dc[p] = kCodesExact ? float4_t{0.f, 0.f, 0.f, 0.f}
                                        : __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[s2][p], kneg,
                                                                                 float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const uint8_t* wr = sl + 1152 * rg + 36 * p;
                        const uint32_t d0 = *reinterpret_cast<const uint32_t*>(wr + wrd);
                        const uint32_t d1 = *reinterpret_cast<const uint32_t*>(wr + wrd + 4);
                        const half_t dv = __builtin_bit_cast(half_t, *reinterpret_cast<const uint16_t*>(wr + drd));
                        const uint32_t p01 = __builtin_amdgcn_perm(d1, d0, sel01);
                        const uint32_t p23 = __builtin_amdgcn_perm(d1, d0, sel23);
                        const half8_t wbv = codes_operand(p01, p23, nu, kneg);
                        const float4_t D = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[s2][p], wbv, dc[p], 0, 0, 0);
                        const float dsc = static_cast<float>(dv);
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[rg][v] = __builtin_fmaf(dsc, D[v], acc[rg][v]);
                    }
                // every LDS read of this slot has returned before the DMA refills it
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (q + NS < Q) {
                    issue();
                    ++issued;
                }
                ++q;
                if (++cslot == NS) cslot = 0;
            }
        }
        finish_tile();
    }
}

template <class C, int MODE>
int launch_q4_xreg(const bx::Target& tg, const uint16_t* x, int K, int64_t batch, int64_t ldx, hipStream_t stream) {
    constexpr size_t lds = C::kLdsBytes;
    const void* fn = reinterpret_cast<const void*>(&gguf_gemv_q4_xreg<C, MODE>);
    if (int rc = prepare_lds(fn, lds)) return rc;
    const int tiles = tg.tile_end[kMaxGroup - 1];
    const int resident = blocks_per_cu(fn, lds, C::kWaves * 64) * cu_count();
    if (resident < 1) return set_error(GDSLLM_ERR_UNSUPPORTED, "gguf_gemv_q4_xreg: no workgroup fits a compute unit");
    const int grid = std::min(tiles, resident);
    hipLaunchKernelGGL((gguf_gemv_q4_xreg<C, MODE>), dim3(grid), dim3(C::kWaves * 64), lds, stream, tg, x, K,
                       static_cast<int>(batch), ldx);
    return check_hip(hipGetLastError(), "gguf_gemv_q4_xreg launch");
}

// Which configuration a launch takes: Half for in_dim <= 4096 with at least
// two 16-row tiles per CU (tiles16: the launch's rows in 16-row tiles; a
// gate/up pair counts both matrices, so it chooses as the group of the two
// does and their sums keep the same bits), else Tall.
inline bool xreg_half(int K, int64_t tiles16) { return K <= 4096 && tiles16 >= 2 * cu_count(); }

template <int MODE>
int launch_xreg(const bx::Target& tg, const uint16_t* x, int K, int64_t batch, int64_t ldx, int64_t tiles16,
                hipStream_t stream) {
    return xreg_half(K, tiles16) ? launch_q4_xreg<bx::Half, MODE>(tg, x, K, batch, ldx, stream)
                                 : launch_q4_xreg<bx::Tall, MODE>(tg, x, K, batch, ldx, stream);
}

// Target of one matrix: tiles of 16 rows.
bx::Target xreg_single(const void* w, void* y, int M, int64_t ldy) {
    bx::Target tg{};
    tg.w[0] = static_cast<const uint8_t*>(w);
    tg.y[0] = static_cast<uint16_t*>(y);
    tg.ldy[0] = ldy;
    tg.m[0] = M;
    for (int i = 0; i < kMaxGroup; ++i) tg.tile_end[i] = (M + bx::kRT - 1) / bx::kRT;
    return tg;
}

// Choice between the two batched Q4_0 kernels.  The x-in-registers kernel
// pays for x before its first weights; it wins where the code kernel's
// 32-row tiles split unevenly over the compute units (896 and 344 tiles on
// 256, which re-read x for every extra tile: 28672x8192 at batch 8 40.4 us
// with the code kernel, 31.7 with it) and where a matrix has at most one
// 16-row tile per compute unit (below), and loses on balanced many-tile
// matrices (8192x8192 at batch 8: 13.6 us with it, 13.3 with the code
// kernel).
inline bool use_q4_xreg(int M, int K) {
    const int t32 = (M + 31) / 32, cu = cu_count();
    return K <= 8192 && t32 > cu && t32 % cu != 0;
}

// Matrices with at most one 16-row tile per compute unit.  Measured on
// MI355X (us, code kernel / x in registers):
//                  batch 4          batch 8
//   1024 x 8192   8.40 / 6.33     8.56 / 8.10
//   2048 x 8192   8.60 / 6.64     8.95 / 8.24
//   4096 x 8192  11.48 / 7.25    11.87 / 8.55
//   4096 x 4096   7.45 / 5.69     7.56 / 7.64
//   1024 x 4096   5.30 / 5.36     5.37 / 7.24
// so it takes in_dim 4097-8192, and in_dim <= 4096 only up to batch 4 with
// more than one tile per two compute units.
inline bool use_q4_xreg_few(int M, int K, int64_t batch) {
    const int t16 = (M + 15) / 16, cu = cu_count();
    if (K > 8192 || t16 > cu) return false;
    if (K > 4096) return true;
    return batch <= 4 && 2 * t16 > cu;
}

// Row-tile height for the code kernel.  A 16-row stage moves 1.8 bytes of x
// per weight byte (a 32-row one 0.9), which costs more than an uneven round
// of 32-row tiles (measured on MI355X: 28672x8192 at batch 8 40.8 us with
// 32-row tiles, 47.1 us with 16; 8192x8192 13.3 vs 15.8 us; 5120x13824 at
// batch 3 / 8 15.3 / 17.8 against 16.7 / 24.2), so 16-row tiles serve only
// matrices of at most one 16-row tile per CU, where 32-row tiles leave CUs
// idle (1024x8192: 8.7 us against 11.6; 4096x11008 at batch 3 / 4 / 8: 8.8 /
// 9.6 / 11.9 against 12.4 / 12.7 / 14.6; 4096x4096 at batch 8: 6.5 against
// 7.8).
inline int q4_codes_rows(int M) { return (M + 15) / 16 <= cu_count() ? 16 : 32; }

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

template <Fmt F, int RT>
int launch_mfma(const void* w, const uint16_t* x, uint16_t* y, int M, int K, int64_t batch, int64_t ldx, int64_t ldy,
                hipStream_t stream) {
    const size_t lds = mfma_lds_bytes<F, RT>();
    const void* fn = reinterpret_cast<const void*>(&gguf_gemv_mfma<F, RT>);
    if (int rc = prepare_lds(fn, lds)) return rc;
    const int tiles = (M + 16 * RT - 1) / (16 * RT);
    const int resident = blocks_per_cu(fn, lds, kMfmaWaves * 64) * cu_count();
    if (resident < 1) return set_error(GDSLLM_ERR_UNSUPPORTED, "gguf_gemv_mfma: no workgroup fits a compute unit");
    const int grid = tiles < resident ? tiles : resident;
    hipLaunchKernelGGL((gguf_gemv_mfma<F, RT>), dim3(grid), dim3(kMfmaWaves * 64), lds, stream,
                       static_cast<const uint8_t*>(w), x, y, M, K, static_cast<int>(batch), ldx, ldy);
    return check_hip(hipGetLastError(), "gguf_gemv_mfma launch");
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
    const int cap = blocks_per_cu(fn, lds, kWaves * 64) * cu_count();
    const int grid = need < cap ? need : cap;
    const bool x_al8 = (reinterpret_cast<uintptr_t>(x) % 8 == 0) && (ldx % 4 == 0);
    hipLaunchKernelGGL((gguf_gemv_staged<F, NB>), dim3(grid), dim3(kWaves * 64), lds, stream,
                       static_cast<const uint8_t*>(w), x, y, M, K, ldx, ldy, x_al8 ? 1 : 0);
    return check_hip(hipGetLastError(), "gguf_gemv launch");
}

// Launch geometry of the row-span kernel: 4-wave workgroups, as many as the
// row groups need (one stage or more per wave), capped at the resident count.
// Measured on MI355X: two stage buffers per wave, or workgroups filling a
// compute unit on their own, lose to more 4-wave workgroups at one buffer
// each.  Returns false when no geometry fits (the caller takes another kernel).
// Sets tg.gb_end: workgroups per matrix, as many as its row groups need while
// all fit at once, else the resident count shared in proportion to row groups.
// Resident workgroups of the row-span kernel with WV waves (0: the LDS does
// not fit), and sets the dynamic LDS size.
template <Fmt F, int NB, int MODE, int WV>
int rows_resident(int NW) {
    const size_t lds = rows_lds_bytes<F, NB>(NW, WV);
    if (lds > static_cast<size_t>(max_lds_bytes())) return 0;
    const void* fn = reinterpret_cast<const void*>(&gguf_gemv_rows<F, NB, MODE, WV>);
    if (prepare_lds(fn, lds) != GDSLLM_OK) return 0;
    return blocks_per_cu(fn, lds, WV * 64) * cu_count();
}

// Split-window plan (MODE 0, NW in 2..4): WV = NW x (1 or 2) row-group
// slots.  Dynamic LDS: the waves' stage buffers, raw x, then the partial row
// sums, tmax stages x WV waves x NB x 4 floats.
template <Fmt F, int NB, int WV>
size_t rows_sw_lds(int NW, int tmax) {
    return rows_lds_bytes<F, NB>(NW, WV) + static_cast<size_t>(tmax) * WV * NB * 4 * sizeof(float);
}

template <Fmt F, int NB, int WV>
int rows_sw_resident(int NW, int tmax) {
    const size_t lds = rows_sw_lds<F, NB, WV>(NW, tmax);
    if (lds > static_cast<size_t>(max_lds_bytes())) return 0;
    const void* fn = reinterpret_cast<const void*>(&gguf_gemv_rows<F, NB, 0, WV, true>);
    if (prepare_lds(fn, lds) != GDSLLM_OK) return 0;
    return blocks_per_cu(fn, lds, WV * 64) * cu_count();
}

// Workgroups of WV = NW * R waves for RG row groups, all resident at once
// (0 if they do not fit); sets tmax, the row groups per slot.
template <Fmt F, int NB, int WV>
int rows_sw_grid(int RG, int NW, int& tmax) {
    if (WV % NW != 0) return 0;
    const int R = WV / NW;
    const int need = (RG + R - 1) / R;
    int grid = std::min(need, rows_sw_resident<F, NB, WV>(NW, 1));
    if (grid <= 0) return 0;
    tmax = (RG + grid * R - 1) / (grid * R);
    if (rows_sw_resident<F, NB, WV>(NW, tmax) < grid) return 0;
    return grid;
}

// Split windows where they put more stages in flight than the plain plan's
// `plain_waves`: sets grid and wv (the wave count, which says which
// instantiation launches), tmax for the LDS size.
template <Fmt F, int NB>
bool plan_split_windows(int RG, int NW, int plain_waves, int& grid, int& wv, int& tmax) {
    if (NW < 2 || NW > 4) return false;
    int best = plain_waves, bg = 0, bw = 0, bt = 0;
    auto consider = [&](int w, int g, int t) {
        if (g > 0 && std::min(g * w, RG * NW) > best) {
            best = std::min(g * w, RG * NW);
            bg = g, bw = w, bt = t;
        }
    };
    int t = 0;
    switch (NW) {
        case 2:
            consider(2, rows_sw_grid<F, NB, 2>(RG, NW, t), t);
            consider(4, rows_sw_grid<F, NB, 4>(RG, NW, t), t);
            break;
        case 3:
            consider(3, rows_sw_grid<F, NB, 3>(RG, NW, t), t);
            consider(6, rows_sw_grid<F, NB, 6>(RG, NW, t), t);
            break;
        default:
            consider(4, rows_sw_grid<F, NB, 4>(RG, NW, t), t);
            consider(8, rows_sw_grid<F, NB, 8>(RG, NW, t), t);
            break;
    }
    if (bg == 0) return false;
    grid = bg, wv = bw, tmax = bt;
    return true;
}

template <Fmt F, int NB, int MODE>
bool plan_rows(RowsTarget& tg, int K, int& grid, int& wv, int& tmax) {
    constexpr bool PAIRED = MODE == 2;
    tmax = 0;
    const int NW = ((K >> 8) + kSbPerWindow - 1) / kSbPerWindow;
    const int parts = PAIRED ? 1 : tg.n;
    int rg_all = 0;
    for (int i = 0; i < parts; ++i)
        rg_all += PAIRED ? (tg.m[0] + 1) / 2 : (tg.m[i] + kRowsPerStage - 1) / kRowsPerStage;
    // 4-wave workgroups, unless 8-wave ones keep more row groups in flight
    // (single matrices whose x fills so much LDS that one 4-wave workgroup
    // fits per CU: the 8192 x 28672 down projection of a 70B layer), or as
    // many where x spans several windows and 8-wave workgroups give every CU
    // one and every wave one row group: x then comes into each CU once
    // instead of once per workgroup (8192 x 8192 at batch 1 / 2: 8.81 /
    // 10.45 against 9.17 / 10.94 us; with several row groups per wave, 28672
    // x 8192 at batch 2, 8-wave workgroups measured no faster)
    wv = kWaves;
    int resident = rows_resident<F, NB, MODE, kWaves>(NW);
    if constexpr (MODE == 0) {
        const int r8 = rows_resident<F, NB, MODE, 8>(NW);
        const int w8 = std::min(r8 * 8, rg_all), w4 = std::min(resident * kWaves, rg_all);
        const bool tie8 = r8 > 0 && w8 == w4 && NW >= 2 && (rg_all + 7) / 8 >= cu_count() && rg_all <= r8 * 8;
        if (w8 > w4 || tie8) {
            wv = 8;
            resident = r8;
        }
    }
    if constexpr (MODE == 2 && F == Fmt::Q4_0 && NB == 1) {
        // Q4_0 pairs at batch 1 over one window whose two-row stages give the
        // resident 4-wave waves more than 1.75 and at most 2 each: one 12-wave
        // workgroup per CU, which loads x into each CU once instead of three
        // times.  Measured (us, 4-wave against 12-wave): 11008 x 4096 (1.79
        // stages per wave) 11.33-11.47 / 10.69-11.11, 12288 x 4096 (2.0)
        // 12.16-12.29 / 11.85-11.89; outside the range 10240 x 4096 (1.67)
        // 10.33-10.57 / 10.56-10.65, 8192 x 4096 8.88 / 9.96, 14336 x 4096
        // 14.16 / 14.90.
        const int w4 = resident * kWaves;
        if (NW == 1 && 4 * rg_all > 7 * w4 && rg_all <= 2 * w4) {
            const int r12 = rows_resident<F, NB, MODE, 12>(NW);
            if (r12 >= cu_count()) {
                wv = 12;
                resident = r12;
            }
        }
    }
    if (resident == 0) return false;
    int need[kMaxGroup], total = 0;
    for (int i = 0; i < parts; ++i) {
        const int rg = PAIRED ? (tg.m[0] + 1) / 2 : (tg.m[i] + kRowsPerStage - 1) / kRowsPerStage;
        need[i] = (rg + wv - 1) / wv;
        total += need[i];
    }
    grid = 0;
    for (int i = 0; i < parts; ++i) {
        int g = need[i];
        if (total > resident) {
            const int rg = PAIRED ? (tg.m[0] + 1) / 2 : (tg.m[i] + kRowsPerStage - 1) / kRowsPerStage;
            g = std::max(rg > 0 ? 1 : 0, static_cast<int>(static_cast<int64_t>(resident) * rg / rg_all));
            g = std::min(g, need[i]);
        }
        grid += g;
        tg.gb_end[i] = grid;
    }
    for (int i = parts; i < kMaxGroup; ++i) tg.gb_end[i] = grid;
    if constexpr (MODE == 0) {
        // one matrix over several windows of x, too few row groups to give
        // every CU a workgroup: split the windows over waves, which spreads
        // the stages over more CUs (tmax > 0 marks the plan).  Where every CU
        // already has a workgroup the split measured slower (4096 x 11008:
        // 9.5 against 8.4 us; more workgroups re-read x from L2 and wait at
        // one more barrier); 1024 x 8192: 4.95 against 5.84 us.
        int g2 = 0, w2 = 0, t2 = 0;
        if (grid > 0 && grid < cu_count() &&
            plan_split_windows<F, NB>(rg_all, NW, std::min(grid * wv, rg_all), g2, w2, t2) && g2 > grid) {
            grid = g2, wv = w2, tmax = t2;
            for (int i = 0; i < kMaxGroup; ++i) tg.gb_end[i] = grid;
        } else if (F == Fmt::Q4_0 && NB == 1 && NW == 2 && rg_all >= 16 * cu_count()) {
            // a long matrix over two windows (28672 x 8192): one 8-wave
            // workgroup per CU, 4 row-group slots x 2 windows, loads x once
            // per CU and never switches windows; 23.9 against 24.6 us for the
            // plain plan's three 4-wave workgroups per CU (8192 x 8192, with
            // fewer row groups per wave, gains nothing)
            const int g8 = rows_sw_grid<F, NB, 8>(rg_all, NW, t2);
            if (g8 > 0) {
                grid = g8, wv = 8, tmax = t2;
                for (int i = 0; i < kMaxGroup; ++i) tg.gb_end[i] = grid;
            }
        }
    }
    // late next-stage issue where it measured faster: gate/up pairs (three
    // 4-wave workgroups per CU) and 8-wave plans; not for 8192 x 8192 (two
    // per CU: 8.94 -> 9.24 us) or single workgroups per CU
    tg.late_issue = MODE == 2 || wv >= 8 ? 1 : 0;
    return grid > 0;
}

template <Fmt F, int NB, int MODE>
int launch_rows(const RowsTarget& tg, const uint16_t* x, int K, int64_t ldx, int grid, int wv, int tmax,
                hipStream_t stream) {
    const int NW = ((K >> 8) + kSbPerWindow - 1) / kSbPerWindow;
    const size_t lds = rows_lds_bytes<F, NB>(NW, wv);
    if constexpr (MODE == 0) {
        if (tmax > 0) {
            auto go = [&](auto wv_c) {
                constexpr int W = decltype(wv_c)::value;
                const size_t sw_lds = rows_sw_lds<F, NB, W>(NW, tmax);
                hipLaunchKernelGGL((gguf_gemv_rows<F, NB, 0, W, true>), dim3(grid), dim3(W * 64), sw_lds, stream, tg,
                                   x, K, ldx);
                return check_hip(hipGetLastError(), "gguf_gemv launch");
            };
            switch (wv) {
                case 2: return go(std::integral_constant<int, 2>{});
                case 3: return go(std::integral_constant<int, 3>{});
                case 4: return go(std::integral_constant<int, 4>{});
                case 6: return go(std::integral_constant<int, 6>{});
                case 8: return go(std::integral_constant<int, 8>{});
                default: return set_error(GDSLLM_ERR_UNSUPPORTED, "gguf_gemv: no split-window kernel for this wave count");
            }
        }
        if (wv == 8) {
            hipLaunchKernelGGL((gguf_gemv_rows<F, NB, MODE, 8>), dim3(grid), dim3(8 * 64), lds, stream, tg, x, K, ldx);
            return check_hip(hipGetLastError(), "gguf_gemv launch");
        }
    }
    if constexpr (MODE == 2 && F == Fmt::Q4_0 && NB == 1) {
        if (wv == 12) {
            hipLaunchKernelGGL((gguf_gemv_rows<F, NB, MODE, 12>), dim3(grid), dim3(12 * 64), lds, stream, tg, x, K,
                               ldx);
            return check_hip(hipGetLastError(), "gguf_gemv launch");
        }
    }
    hipLaunchKernelGGL((gguf_gemv_rows<F, NB, MODE>), dim3(grid), dim3(kWaves * 64), lds, stream, tg, x, K, ldx);
    return check_hip(hipGetLastError(), "gguf_gemv launch");
}

// The row-span kernel serves batch <= 2 with in_dim % 256 == 0 (in_dim <=
// 2^20), 16-byte aligned weights, x 16-byte aligned with ldx % 8 == 0.
// Returns GDSLLM_OK after launching, -1 when the request does not qualify (or
// no geometry fits), else an error code.
template <Fmt F, int MODE>
int try_rows(RowsTarget tg, const void* x, int K, int64_t batch, int64_t ldx, hipStream_t s) {
    bool w_al16 = true;
    for (int i = 0; i < tg.n; ++i) w_al16 = w_al16 && reinterpret_cast<uintptr_t>(tg.w[i]) % 16 == 0;
    const bool x_al16 = reinterpret_cast<uintptr_t>(x) % 16 == 0 && (ldx % 8 == 0 || batch == 1);
    if (batch > 2 || K % 256 != 0 || K > (1 << 20) || !w_al16 || !x_al16) return -1;
    const auto* xp = static_cast<const uint16_t*>(x);
    int grid = 0, wv = kWaves, tmax = 0;
    if (batch == 1) {
        if (!plan_rows<F, 1, MODE>(tg, K, grid, wv, tmax)) return -1;
        return launch_rows<F, 1, MODE>(tg, xp, K, ldx, grid, wv, tmax, s);
    }
    if (!plan_rows<F, 2, MODE>(tg, K, grid, wv, tmax)) return -1;
    return launch_rows<F, 2, MODE>(tg, xp, K, ldx, grid, wv, tmax, s);
}

RowsTarget single_target(const void* w, void* y, int M, int64_t ldy) {
    RowsTarget tg{};
    tg.w[0] = static_cast<const uint8_t*>(w);
    tg.y[0] = static_cast<uint16_t*>(y);
    tg.ldy[0] = ldy;
    tg.m[0] = M;
    tg.n = 1;
    return tg;
}

// Shape checks shared by the GEMV entry points.
int check_gemv_args(const std::string& n, int64_t out_dim, int64_t in_dim, int64_t batch) {
    if (out_dim < 0 || in_dim < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (in_dim % 32 != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         n + ": in_dim must be a multiple of 32, got " + std::to_string(in_dim));
    if (batch < 1 || batch > 8)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": batch must be in [1, 8], got " + std::to_string(batch));
    if (out_dim > (int64_t(1) << 30) || in_dim > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    return GDSLLM_OK;
}

template <Fmt F>
int gemv(const char* name, const void* w, const void* x, void* y, int64_t out_dim, int64_t in_dim,
         int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    const std::string n(name);
    if (int rc = check_gemv_args(n, out_dim, in_dim, batch)) return rc;
    if (out_dim == 0 || in_dim == 0) return ok();  // silent no-op, as the reference launchers
    if (!w || !x || !y) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (batch > 1 && (ldx < in_dim || ldy < out_dim))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than the row length");
    if (reinterpret_cast<uintptr_t>(x) % 2 || reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": x and y must be 2-byte aligned");
    hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(out_dim), K = static_cast<int>(in_dim);
    const auto* xp = static_cast<const uint16_t*>(x);
    auto* yp = static_cast<uint16_t*>(y);
    const bool fast = (K % 256 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    const bool x_al16 = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (ldx % 8 == 0);
    // Q4_0 at batch 2 whose two rows of x would fill more than 64 KiB of the
    // row-span kernel's LDS (8192 x 28672: 112 KiB, one 4-wave workgroup per
    // CU, 37.0 us) goes to the code kernel (30.5 us); below that the row-span
    // kernel is faster (11008 x 4096: 9.3 against 13.7 us)
    const bool b2_codes = F == Fmt::Q4_0 && batch == 2 && fast && x_al16 && K <= (1 << 20) &&
                          rows_xraw_bytes(2, ((K >> 8) + kSbPerWindow - 1) / kSbPerWindow) > 65536;
    int rc = b2_codes ? -1 : try_rows<F, 0>(single_target(w, y, M, ldy), x, K, batch, ldx, s);
    if (rc != -1) return rc == GDSLLM_OK ? ok() : rc;
    rc = GDSLLM_OK;
    if (F == Fmt::Q4_0 && fast && batch >= 3 && x_al16 && (use_q4_xreg(M, K) || use_q4_xreg_few(M, K, batch)) &&
        2 * (7 * ldx + K) < (int64_t{1} << 31)) {
        const int rc2 = launch_xreg<0>(xreg_single(w, y, M, ldy), xp, K, batch, ldx, (M + 15) / 16, s);
        return rc2 == GDSLLM_OK ? ok() : rc2;
    }
    if (F == Fmt::Q4_0 && fast && (batch >= 3 || b2_codes) && K <= (1 << 20) && x_al16) {
        const bool x2 = batch <= 4;  // x rows 0-3 in two transfers per stage
        const int rc2 = q4_codes_rows(M) == 32
                            ? (x2 ? launch_q4_codes<32, 2>(w, xp, yp, M, K, batch, ldx, ldy, s)
                                  : launch_q4_codes<32, 4>(w, xp, yp, M, K, batch, ldx, ldy, s))
                            : (x2 ? launch_q4_codes<16, 2>(w, xp, yp, M, K, batch, ldx, ldy, s)
                                  : launch_q4_codes<16, 4>(w, xp, yp, M, K, batch, ldx, ldy, s));
        return rc2 == GDSLLM_OK ? ok() : rc2;
    }
    if (fast && batch >= 3 && K <= (1 << 20) && x_al16) {
        // Q8_0 (Q4_0 took the code kernels above)
        const int rc2 = launch_mfma<F, 1>(w, xp, yp, M, K, batch, ldx, ldy, s);
        return rc2 == GDSLLM_OK ? ok() : rc2;
    }
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

// Batch 3-8 launches of the x-in-registers kernel over several matrices
// (groups, gate/up pairs): in_dim a multiple of 256 up to 8192 (one slice of
// x per wave), 16-byte aligned weights and x rows, x offsets within 2^31.
bool xreg_fits(const uint8_t* const* w, int n, const void* x, int64_t K, int64_t batch, int64_t ldx) {
    if (batch < 3 || K % 256 != 0 || K > 8192 || reinterpret_cast<uintptr_t>(x) % 16 != 0 || ldx % 8 != 0 ||
        2 * (7 * ldx + K) >= (int64_t{1} << 31))
        return false;
    for (int i = 0; i < n; ++i)
        if (reinterpret_cast<uintptr_t>(w[i]) % 16 != 0) return false;
    return true;
}

// n matrices sharing x (q/k/v of one layer): one launch when the row-span
// kernel (batch 1-2) or the x-in-registers kernel (Q4_0, batch 3-8) serves
// the shape, else one GEMV per matrix.
template <Fmt F>
int gemv_group(const char* name, int n, const void* const* w, void* const* y, const int64_t* out_dims,
               const void* x, int64_t in_dim, int64_t batch, int64_t ldx, void* stream) {
    const std::string nm(name);
    if (n < 1 || n > kMaxGroup)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": n must be in [1, 4], got " + std::to_string(n));
    if (!w || !y || !out_dims) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": null pointer");
    RowsTarget tg{};
    tg.n = n;
    bool any = false;
    for (int i = 0; i < n; ++i) {
        if (int rc = check_gemv_args(nm, out_dims[i], in_dim, batch)) return rc;
        if (out_dims[i] > 0 && in_dim > 0 && (!w[i] || !y[i] || !x))
            return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": null pointer");
        if (reinterpret_cast<uintptr_t>(y[i]) % 2) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": y must be 2-byte aligned");
        any = any || out_dims[i] > 0;
        tg.w[i] = static_cast<const uint8_t*>(w[i]);
        tg.y[i] = static_cast<uint16_t*>(y[i]);
        tg.ldy[i] = out_dims[i];
        tg.m[i] = static_cast<int>(out_dims[i]);
    }
    if (!any || in_dim == 0) return ok();
    if (batch > 1 && ldx < in_dim) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": ldx smaller than in_dim");
    if (reinterpret_cast<uintptr_t>(x) % 2) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": x must be 2-byte aligned");
    const int rc = n == 1 ? try_rows<F, 0>(tg, x, static_cast<int>(in_dim), batch, ldx, as_stream(stream))
                          : try_rows<F, 1>(tg, x, static_cast<int>(in_dim), batch, ldx, as_stream(stream));
    if (rc != -1) return rc == GDSLLM_OK ? ok() : rc;
    if (F == Fmt::Q4_0 && n > 1 && xreg_fits(tg.w, n, x, in_dim, batch, ldx)) {
        // batch 3-8: the x-in-registers kernel over the matrices' 16-row tiles
        bx::Target xt{};
        int tiles = 0;
        for (int i = 0; i < n; ++i) {
            xt.w[i] = tg.w[i], xt.y[i] = tg.y[i], xt.ldy[i] = tg.ldy[i], xt.m[i] = tg.m[i];
            tiles += (tg.m[i] + bx::kRT - 1) / bx::kRT;
            xt.tile_end[i] = tiles;
        }
        for (int i = n; i < kMaxGroup; ++i) xt.tile_end[i] = tiles;
        const int rc2 = launch_xreg<1>(xt, static_cast<const uint16_t*>(x), static_cast<int>(in_dim), batch, ldx,
                                       tiles, as_stream(stream));
        return rc2 == GDSLLM_OK ? ok() : rc2;
    }
    for (int i = 0; i < n; ++i)
        if (int e = gemv<F>(name, w[i], x, y[i], out_dims[i], in_dim, batch, ldx, out_dims[i], stream)) return e;
    return ok();
}

// h = fp16(silu(gate x) * (up x)) in one launch (gate/up pairing in the
// row-span kernel at batch 1-2, in the x-in-registers kernel for Q4_0 at
// batch 3-8).
template <Fmt F>
int gate_up_silu(const char* name, const void* w_gate, const void* w_up, const void* x, void* h, int64_t out_dim,
                 int64_t in_dim, int64_t batch, int64_t ldx, int64_t ldh, void* stream) {
    const std::string nm(name);
    if (int rc = check_gemv_args(nm, out_dim, in_dim, batch)) return rc;
    if (out_dim == 0 || in_dim == 0) return ok();
    if (!w_gate || !w_up || !x || !h) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": null pointer");
    if (batch > 1 && (ldx < in_dim || ldh < out_dim))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": ldx/ldh smaller than the row length");
    if (reinterpret_cast<uintptr_t>(h) % 2) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, nm + ": h must be 2-byte aligned");
    RowsTarget tg{};
    tg.n = 2;
    tg.w[0] = static_cast<const uint8_t*>(w_gate);
    tg.w[1] = static_cast<const uint8_t*>(w_up);
    tg.y[0] = static_cast<uint16_t*>(h);
    tg.ldy[0] = ldh;
    tg.m[0] = tg.m[1] = static_cast<int>(out_dim);
    int rc = try_rows<F, 2>(tg, x, static_cast<int>(in_dim), batch, ldx, as_stream(stream));
    if (rc == -1 && F == Fmt::Q4_0 && xreg_fits(tg.w, 2, x, in_dim, batch, ldx)) {
        // batch 3-8: the x-in-registers kernel, 8 gate and 8 up rows per tile
        bx::Target xt{};
        xt.w[0] = tg.w[0], xt.w[1] = tg.w[1], xt.y[0] = tg.y[0], xt.ldy[0] = ldh, xt.m[0] = static_cast<int>(out_dim);
        for (int i = 0; i < kMaxGroup; ++i) xt.tile_end[i] = static_cast<int>((out_dim + bx::kRT / 2 - 1) / (bx::kRT / 2));
        rc = launch_xreg<2>(xt, static_cast<const uint16_t*>(x), static_cast<int>(in_dim), batch, ldx,
                            2 * ((out_dim + bx::kRT - 1) / bx::kRT), as_stream(stream));
    }
    if (rc == -1)
        return set_error(GDSLLM_ERR_UNSUPPORTED,
                         nm + ": needs in_dim % 256 == 0, 16-byte aligned weights and x (ldx % 8 == 0), and for "
                              "batch 3-8 Q4_0 with in_dim <= 8192");
    return rc == GDSLLM_OK ? ok() : rc;
}

}  // namespace
}  // namespace gdsllm

using namespace gdsllm;

extern "C" int gdsllm_fused_q4_0_gemv_group(int n, const void* const* weights, void* const* ys,
                                            const int64_t* out_dims, const void* x, int64_t in_dim, int64_t batch,
                                            int64_t ldx, void* stream) {
    return gemv_group<Fmt::Q4_0>("fused_q4_0_gemv_group", n, weights, ys, out_dims, x, in_dim, batch, ldx, stream);
}

extern "C" int gdsllm_fused_q8_0_gemv_group(int n, const void* const* weights, void* const* ys,
                                            const int64_t* out_dims, const void* x, int64_t in_dim, int64_t batch,
                                            int64_t ldx, void* stream) {
    return gemv_group<Fmt::Q8_0>("fused_q8_0_gemv_group", n, weights, ys, out_dims, x, in_dim, batch, ldx, stream);
}

extern "C" int gdsllm_fused_q4_0_gate_up_silu(const void* w_gate, const void* w_up, const void* x, void* h,
                                              int64_t out_dim, int64_t in_dim, int64_t batch, int64_t ldx,
                                              int64_t ldh, void* stream) {
    return gate_up_silu<Fmt::Q4_0>("fused_q4_0_gate_up_silu", w_gate, w_up, x, h, out_dim, in_dim, batch, ldx, ldh,
                                   stream);
}

extern "C" int gdsllm_fused_q8_0_gate_up_silu(const void* w_gate, const void* w_up, const void* x, void* h,
                                              int64_t out_dim, int64_t in_dim, int64_t batch, int64_t ldx,
                                              int64_t ldh, void* stream) {
    return gate_up_silu<Fmt::Q8_0>("fused_q8_0_gate_up_silu", w_gate, w_up, x, h, out_dim, in_dim, batch, ldx, ldh,
                                   stream);
}

extern "C" int gdsllm_fused_q4_0_gemv(const void* weight, const void* x, void* y, int64_t out_dim,
                                      int64_t in_dim, int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    return gemv<Fmt::Q4_0>("fused_q4_0_gemv", weight, x, y, out_dim, in_dim, batch, ldx, ldy, stream);
}

extern "C" int gdsllm_fused_q8_0_gemv(const void* weight, const void* x, void* y, int64_t out_dim,
                                      int64_t in_dim, int64_t batch, int64_t ldx, int64_t ldy, void* stream) {
    return gemv<Fmt::Q8_0>("fused_q8_0_gemv", weight, x, y, out_dim, in_dim, batch, ldx, ldy, stream);
}
