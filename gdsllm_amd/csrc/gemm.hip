// Prefill dequant-GEMM for GGUF Q4_0 weights whose in_dim is not a multiple
// of 256 (the split-K kernel family of prefill.hip serves every other shape).
//
// Y[t][r] = fp16( sum_k X[t][k] * W[r][k] ) for a chunk of T prompt tokens:
// what the reference's prefill branch computes as dequant -> F.linear
// (runtime/llama.py:160-166), fused so the fp16 weight matrix never goes back
// to HBM.  W enters the matrix cores as the bit-exact fp16 dequantized value
// d*(q-8) (the same fp16 tensor the reference hands to cuBLAS), X as fp16,
// accumulation in fp32 (v_mfma_f32_16x16x32_f16), one fp16 rounding at the end.
//
// Workgroup tile: BT = 2*TW tokens x 128 weight rows, 4 waves in a 2 x 2
// grid, each wave TW tokens x 64 rows (TW/16 x 4 MFMA fragments).  K advances
// one Q4_0 block (32 elements) per step:
//  * X: 16-byte DMA transfers (global_load_lds) into a ring of kXRing tiles.
//    Slot 4t + (c ^ ((t >> 1) & 3)) of a tile holds elements 8c..8c+7 of
//    token t, so the 16 lanes reading chunk c of 16 consecutive tokens hit 8
//    distinct 16-byte bank groups twice (no conflicts beyond the hardware's
//    two-pass b128 read).
//  * W: the 18-byte block of each of the 128 rows comes in as the two aligned
//    16-byte chunks that contain it (DMA, ring of kWRing steps, which runs
//    kWRing - kXRing steps ahead of X), is dequantized bit-exactly by the
//    workgroup (two threads per row, one half-block each) into a padded fp16
//    tile (80-byte rows: conflict-free fragment reads), double-buffered.
//  * Transfers of one step form a bundle of fixed size per wave (dummies past
//    the end), so the waits are compile-time vmcnt counts: the compiler does
//    not count LDS-DMA transfers itself.
// Per step: wait for the step's bundle, barrier, issue the bundle kXRing - 1
// steps ahead, dequantize this step's W, barrier, then 32 (TW = 128) MFMAs.
// LDS is read and written with the raw helpers: a compiler-visible LDS access
// would wait for every transfer in flight.
//
// MFMA operand layout (16x16x32 f16): lane l holds A row (l % 16) and B column
// (l % 16), eight consecutive k values 8*(l/16)..+7 of each; the result holds
// D[4*(l/16) + v][l % 16] in its four fp32 registers.

#include "common.h"

namespace gdsllm {
namespace {

constexpr int kGemmWaves = 4;
constexpr int kGemmRows = 128;   // weight rows per workgroup (2 waves x 64)
constexpr int kXRing = 4;        // X tiles in flight / in use
constexpr int kWRing = 8;        // raw W steps in flight / in use
constexpr int kWRowBytes = 80;   // fp16 W tile row: 32 values + 16 bytes of padding

template <int TW>
struct GemmShape {
    static constexpr int BT = 2 * TW;               // tokens per workgroup
    static constexpr int kXTile = BT * 64;          // bytes: BT tokens x 32 fp16
    static constexpr int kXPerWave = BT * 4 / 64 / kGemmWaves;  // X transfers per wave per step
    static constexpr int kWRaw = kGemmRows * 32;    // bytes: two 16-byte chunks per row
    static constexpr int kWTile = kGemmRows * kWRowBytes;
    static constexpr int kBundle = kXPerWave + 1;   // transfers per wave per step
    static constexpr int kLds = kXRing * kXTile + kWRing * kWRaw + 2 * kWTile;
    static_assert(kXPerWave * 64 * kGemmWaves == BT * 4, "X tile splits evenly over the waves");
    static_assert(kGemmRows * 2 == 64 * kGemmWaves, "one raw-W transfer per wave per step");
};

template <int TW>
__global__ __launch_bounds__(kGemmWaves * 64) void dequant_gemm_q4_0(const uint8_t* __restrict__ W,
                                                                     const uint16_t* __restrict__ X,
                                                                     uint16_t* __restrict__ Y, int M, int K, int T,
                                                                     int64_t ldx, int64_t ldy) {
    using G = GemmShape<TW>;
    constexpr int kFragT = TW / 16, kFragM = 4;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* xring = lds;
    uint8_t* wraw = lds + kXRing * G::kXTile;
    uint8_t* wtile = wraw + kWRing * G::kWRaw;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wt = wave >> 1, wm = wave & 1;
    const int t0 = blockIdx.y * G::BT, m0 = blockIdx.x * kGemmRows;
    const int64_t row_bytes = static_cast<int64_t>(K >> 5) * 18;
    const int nsteps = K >> 5;

    // This lane's X sources: transfer i of this wave fills slot s = 64*(wave*kXPerWave + i) + lane.
    const uint16_t* xsrc[G::kXPerWave];
#pragma unroll
    for (int i = 0; i < G::kXPerWave; ++i) {
        const int s = 64 * (wave * G::kXPerWave + i) + lane;
        const int t = s >> 2, c = (s & 3) ^ ((t >> 1) & 3);
        xsrc[i] = t0 + t < T ? X + static_cast<int64_t>(t0 + t) * ldx + 8 * c : X;
    }
    // This lane's W source: slot 64*wave + lane = chunk (s & 1) of row s >> 1.
    const int wr = (64 * wave + lane) >> 1, wpart = lane & 1;
    const uint8_t* wrow = W + static_cast<int64_t>(m0 + wr < M ? m0 + wr : m0) * row_bytes;

    auto issue_x = [&](int step) {
        const bool live = step < nsteps;
        uint8_t* dst = xring + (step % kXRing) * G::kXTile + 1024 * (wave * G::kXPerWave);
#pragma unroll
        for (int i = 0; i < G::kXPerWave; ++i) dma16_cached(live ? xsrc[i] + 32 * step : X, dst + 1024 * i);
    };
    auto issue_w = [&](int step) {
        const bool live = step < nsteps;
        const uintptr_t a = reinterpret_cast<uintptr_t>(wrow + 18 * static_cast<int64_t>(live ? step : 0));
        const uint8_t* src = reinterpret_cast<const uint8_t*>((a & ~uintptr_t(15)) + 16 * wpart);
        dma16(src, wraw + (step % kWRing) * G::kWRaw + 1024 * wave);
    };

    // Pre-bundles: raw W for steps 0 .. kWRing-kXRing-1; then bundles 0 .. kXRing-2.
    for (int j = 0; j < kWRing - kXRing; ++j) issue_w(j);
    for (int b = 0; b < kXRing - 1; ++b) {
        issue_x(b);
        issue_w(b + kWRing - kXRing);
    }

    // dequantization role: row dr, half dh (elements 16*dh .. 16*dh+15)
    const int dr = tid >> 1, dh = tid & 1;
    const int64_t drow_off = static_cast<int64_t>(m0 + dr) * row_bytes;
    const uint32_t dmask = dh ? 0x00F000F0u : 0x000F000Fu, dbits = dh ? 0x54005400u : 0x64006400u;
    const half2_t doff = dh ? half2_t{static_cast<half_t>(-72.0f), static_cast<half_t>(-72.0f)}
                            : half2_t{static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f)};

    float4_t acc[kFragT][kFragM];
#pragma unroll
    for (int a = 0; a < kFragT; ++a)
#pragma unroll
        for (int b = 0; b < kFragM; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int fi = lane & 15, fg = lane >> 4;
    // A fragment reads: token (wt*TW + 16a + fi), chunk fg -> swizzled slot
    uint32_t xoff[kFragT];
#pragma unroll
    for (int a = 0; a < kFragT; ++a) {
        const int t = wt * TW + 16 * a + fi;
        xoff[a] = 16 * (4 * t + (fg ^ ((t >> 1) & 3)));
    }
    const uint32_t woff = (wm * 64 + fi) * kWRowBytes + 16 * fg;

    for (int s = 0; s < nsteps; ++s) {
        // bundle s (X of step s, raw W of step s + kWRing - kXRing) has landed
        wait_vmcnt<(kXRing - 2) * G::kBundle>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_x(s + kXRing - 1);
        issue_w(s + kWRing - 1);

        // dequantize step s: the 18-byte block sits at byte (row offset + 18s) % 16
        // of the row's two raw chunks; 6 dwords from there cover it
        {
            const uint32_t o = static_cast<uint32_t>((drow_off + 18 * static_cast<int64_t>(s)) & 15);
            const uint32_t base = lds_addr(wraw + (s % kWRing) * G::kWRaw + 32 * dr + (o & ~3u));
            uint64_t rp[3];
            lds_read4x6_sync(base, rp);
            uint32_t r[6];
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                r[2 * i] = static_cast<uint32_t>(rp[i]);
                r[2 * i + 1] = static_cast<uint32_t>(rp[i] >> 32);
            }
            const uint32_t sh = o & 3u;
            uint32_t b[5];  // bytes o .. o+19 of the raw chunks
#pragma unroll
            for (int i = 0; i < 5; ++i) b[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], sh);
            const half_t dv = __builtin_bit_cast(half_t, static_cast<uint16_t>(b[0] & 0xFFFFu));
            const half2_t dd = {dv, dv};
            uint32_t q[4];  // qs bytes 0..15 = bytes 2..17
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = align2(b[i], b[i + 1]);
            uint32_t outv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // (b0, b1) and (b2, b3) into the low byte of each half, natural k order
                const uint32_t t01 = __builtin_amdgcn_perm(0u, q[i], 0x0C010C00u);
                const uint32_t t23 = __builtin_amdgcn_perm(0u, q[i], 0x0C030C02u);
                const half2_t p01 = __builtin_bit_cast(half2_t, (t01 & dmask) | dbits) + doff;  // exact q - 8
                const half2_t p23 = __builtin_bit_cast(half2_t, (t23 & dmask) | dbits) + doff;
                outv[2 * i] = __builtin_bit_cast(uint32_t, p01 * dd);  // one RNE rounding
                outv[2 * i + 1] = __builtin_bit_cast(uint32_t, p23 * dd);
            }
            const uint32_t dst = lds_addr(wtile + (s & 1) * G::kWTile + dr * kWRowBytes + 32 * dh);
            lds_write16_raw(dst, u32x4_t{outv[0], outv[1], outv[2], outv[3]});
            lds_write16_raw(dst + 16, u32x4_t{outv[4], outv[5], outv[6], outv[7]});
        }
        lds_barrier();

        const uint8_t* xt = xring + (s % kXRing) * G::kXTile;
        const uint32_t wt_ = lds_addr(wtile + (s & 1) * G::kWTile) + woff;
        u32x4_t bv[kFragM];
        lds_read16x4_sync<16 * kWRowBytes>(wt_, bv);
        half8_t bf[kFragM];
#pragma unroll
        for (int b = 0; b < kFragM; ++b) bf[b] = __builtin_bit_cast(half8_t, bv[b]);
#pragma unroll
        for (int a = 0; a < kFragT; ++a) {
            const half8_t af = __builtin_bit_cast(half8_t, lds_read16_sync(lds_addr(xt + xoff[a])));
#pragma unroll
            for (int b = 0; b < kFragM; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[a][b], 0, 0, 0);
        }
    }
    // no transfer into this workgroup's LDS may outlive it
    wait_vmcnt<0>();

#pragma unroll
    for (int a = 0; a < kFragT; ++a)
#pragma unroll
        for (int b = 0; b < kFragM; ++b) {
            const int m = m0 + wm * 64 + 16 * b + fi;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int t = t0 + wt * TW + 16 * a + 4 * fg + v;
                if (t < T && m < M) Y[t * ldy + m] = f2h_bits(acc[a][b][v]);
            }
        }
}

template <int TW>
int launch_gemm(const void* w, const void* x, void* y, int M, int K, int T, int64_t ldx, int64_t ldy,
                hipStream_t stream) {
    using G = GemmShape<TW>;
    const void* fn = reinterpret_cast<const void*>(&dequant_gemm_q4_0<TW>);
    if (int rc = prepare_lds(fn, G::kLds)) return rc;
    // token tiles go in grid.y; long prompts are split into launches of at most
    // kMaxTileRows tiles each so the y dimension stays within the hardware limit
    constexpr int kMaxTileRows = 32768;
    const unsigned row_tiles = static_cast<unsigned>((M + kGemmRows - 1) / kGemmRows);
    for (int t = 0; t < T; t += kMaxTileRows * G::BT) {
        const int tc = std::min(T - t, kMaxTileRows * G::BT);
        dim3 grid(row_tiles, static_cast<unsigned>((tc + G::BT - 1) / G::BT));
        hipLaunchKernelGGL((dequant_gemm_q4_0<TW>), grid, dim3(kGemmWaves * 64), G::kLds, stream,
                           static_cast<const uint8_t*>(w), static_cast<const uint16_t*>(x) + t * ldx,
                           static_cast<uint16_t*>(y) + t * ldy, M, K, tc, ldx, ldy);
        if (int rc = check_hip(hipGetLastError(), "dequant_gemm_q4_0 launch")) return rc;
    }
    return GDSLLM_OK;
}

}  // namespace

// Q4_0 prefill GEMM for in_dim % 32 == 0 off the split-K kernels' grid
// (in_dim % 256 != 0): one Q4_0 block per K step.  Arguments are validated by
// the caller (gdsllm_dequant_gemm_q4_0).  Wider token tiles dequantize each
// weight block fewer times, but a small problem needs the narrower tiles to
// give every CU a workgroup: take the widest tile (256, 128 or 64 tokens)
// that still does.
int dequant_gemm_q4_0_blockwise(const void* weight, const void* x, void* y, int M, int K, int T, int64_t ldx,
                                int64_t ldy, hipStream_t st) {
    const int64_t row_tiles = (M + kGemmRows - 1) / kGemmRows;
    auto tiles = [&](int bt) { return row_tiles * ((T + bt - 1) / bt); };
    return tiles(256) >= cu_count()   ? launch_gemm<128>(weight, x, y, M, K, T, ldx, ldy, st)
           : tiles(128) >= cu_count() ? launch_gemm<64>(weight, x, y, M, K, T, ldx, ldy, st)
                                      : launch_gemm<32>(weight, x, y, M, K, T, ldx, ldy, st);
}

}  // namespace gdsllm
