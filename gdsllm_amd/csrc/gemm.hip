// Prefill dequant-GEMM for GGUF Q4_0 weights on the gfx950 matrix cores.
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

// ---------------------------------------------------------------------------
// Split-K workgroup GEMM for in_dim % 256 == 0 (every LLaMA projection).
//
// Workgroup tile: 128 weight rows x 64 tokens, 8 waves (two per SIMD).  A
// stage is 128 values of k (4 Q4_0 blocks); wave w multiplies block w & 3 of
// every stage for weight rows 64*(w >> 2) .. +63 and all 64 tokens, so each
// weight is dequantized exactly once per workgroup, in registers, straight
// from its raw 18-byte block (no fp16 weight tile).  At the end the four
// K-quarters of each output are summed through LDS in a fixed order, so the
// result does not depend on timing.
//
//  * MFMA v_mfma_f32_32x32x16_f16, A = X (32 tokens x 16 k), B = W (16 k x 32
//    rows).  Lane l holds token/row l % 32 and k values 8(l/32) .. +7 of a
//    16-value k-step.  K-step 0 of a block is elements 0..15 = low nibbles of
//    qs[0..15], k-step 1 elements 16..31 = high nibbles: lane half h reads
//    qs[8h .. 8h+7] once and feeds both k-steps (low, then high nibbles).
//  * Dequant is the reference's value bit for bit: (q | 0x6400) = 1024+q and
//    (q<<4 | 0x5400) = 64+q are exact fp16, minus 1032 / 72 gives q-8 exactly,
//    one packed multiply by d rounds once (gguf_dequant.cu:105-106).
//  * Data path: global -> LDS by DMA (global_load_lds), X in a ring of 5
//    stages (16 KiB each), W in a ring of 4 super-blocks (128 rows x 144 B =
//    18 transfers of 1 KiB: waves 0-5 issue 3 each, waves 6-7 three 4-byte
//    dummies into a scratch word so every wave counts 3).  At stage s a
//    wave issues X of stage s+4 and, on even s, super-block s/2+3; reads and
//    dequantizes the operands of stage s+1; and runs the 8 MFMAs of stage s.
//    One LDS barrier per stage.  The DMA is issued from inline assembly, so
//    the compiler neither sees nor waits for it: the vmcnt waits are written
//    out (every vector-memory operation in the loop is one of these
//    transfers, so the counts are exact), and every LDS read is an ordinary
//    instruction the compiler schedules around the MFMAs.
//  * X tile layout: token t's 16 chunks of 16 bytes (8 values) sit in one
//    256-byte row, chunk c at position c ^ (t & 15): the lanes reading chunk c
//    of 32 consecutive tokens hit distinct 16-byte bank groups.
//  * Workgroups are remapped so that each XCD (dispatch goes round-robin over
//    the 8 XCDs) takes a contiguous range of tiles, token tile major: its L2
//    holds one or two X token tiles while it streams its own weight rows.
namespace sk {
constexpr int kWaves = 8;
constexpr int kBM = 128;                    // weight rows per workgroup
constexpr int kBT = 64;                     // tokens per workgroup
constexpr int kStageK = 128;                // k values per stage
constexpr int kXRing = 5;
constexpr int kWRing = 4;
constexpr int kXSlot = kBT * kStageK * 2;   // 16384 bytes
constexpr int kWSlot = kBM * 144;           // 18432 bytes: one super-block of 128 rows
constexpr int kWOff = kXRing * kXSlot;
constexpr int kDummyOff = kXRing * kXSlot + kWRing * kWSlot;
constexpr int kLds = kDummyOff + 256;       // 155904
constexpr int kRegion = 16384;              // one wave's 64 accumulators x 64 lanes x 4 bytes
static_assert(kWaves * kRegion <= kLds, "reduction fits in the ring");
static_assert(kXSlot / 1024 == 2 * kWaves, "two 16-byte X transfers per wave per stage");
static_assert(kWSlot / 1024 == 3 * (kWaves - 2), "waves 0-5 move a super-block in three transfers each");
}  // namespace sk

typedef float float16_t __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(sk::kWaves * 64) void dequant_gemm_q4_0_sk(const uint8_t* __restrict__ W,
                                                                      const uint16_t* __restrict__ X,
                                                                      uint16_t* __restrict__ Y, int M, int K, int T,
                                                                      int64_t ldx, int64_t ldy, int mtiles) {
    using namespace sk;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int kq = wave & 3, rq = wave >> 2;

    // XCD-aware tile order: dispatch sends workgroup b to XCD b % 8.
    const int nwg = gridDim.x, b = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = b & 7;
    const int q = xcd * per + (xcd < rem ? xcd : rem) + (b >> 3);
    const int m0 = (q % mtiles) * kBM, t0 = (q / mtiles) * kBT;

    const int64_t row_bytes = static_cast<int64_t>(K >> 5) * 18;
    const int nst = K / kStageK, nsb = nst >> 1;
    const uint32_t lds0 = lds_addr(lds);

    // ---- DMA sources: a wave-uniform base per stage (scalar arithmetic) plus
    // a fixed 32-bit byte offset per lane.  X transfer i (0..15) fills 16-byte
    // slot 64i + l of a stage: token 4i + l/16, chunk (l & 15) ^ (token & 15).
    // Wave w issues i = 2w, 2w+1.  Tokens past T read token T-1.
    const uint16_t* xtile = X + static_cast<int64_t>(t0) * ldx;
    uint32_t xoff[2];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int t = 4 * (2 * wave + ii) + (lane >> 4);
        const int c = (lane & 15) ^ (t & 15);
        const int tl = t0 + t < T ? t : T - 1 - t0;
        xoff[ii] = static_cast<uint32_t>(2 * (static_cast<int64_t>(tl) * ldx + 8 * c));
    }
    // W transfer i (0..17) moves 16-byte piece g = 64i + l of a super-block:
    // row g / 9, bytes 16 (g % 9) of the row's 144.  Wave w < 6 issues
    // i = 3w .. 3w+2.  Rows past M read row M-1.
    const bool w_real = wave < 6;
    const uint8_t* wtile = W + static_cast<int64_t>(m0) * row_bytes;
    uint32_t woff[3];
#pragma unroll
    for (int ii = 0; ii < 3; ++ii) {
        const int g = 64 * (3 * (w_real ? wave : 0) + ii) + lane;
        const int rl = m0 + g / 9 < M ? g / 9 : M - 1 - m0;
        woff[ii] = static_cast<uint32_t>(static_cast<int64_t>(rl) * row_bytes + 16 * (g % 9));
    }
    // Stage / super-block indices past the end are clamped to the last one:
    // the same number of transfers (the waits count them) into a slot no
    // later stage reads.
    auto issue_x = [&](int st) {
        const uint32_t dst = lds0 + (st % sk::kXRing) * kXSlot + 1024 * (2 * wave);
        const uint16_t* base = xtile + kStageK * (st < nst ? st : nst - 1);
        dma16_asm(xoff[0], base, dst);
        dma16_asm(xoff[1], base, dst + 1024);
    };
    auto issue_w = [&](int sb) {
        if (w_real) {
            const uint32_t dst = lds0 + kWOff + (sb % sk::kWRing) * kWSlot + 1024 * (3 * wave);
            const uint8_t* base = wtile + 144 * (sb < nsb ? sb : nsb - 1);
            dma16_asm(woff[0], base, dst);
            dma16_asm(woff[1], base, dst + 1024);
            dma16_asm(woff[2], base, dst + 2048);
        } else {
            const uint32_t dst = lds0 + kDummyOff;
            dma4_asm(0u, W, dst);
            dma4_asm(0u, W, dst);
            dma4_asm(0u, W, dst);
        }
    };

    // ---- operand reads (stage u: block jj = 4(u&1) + kq of super-block u/2)
    uint32_t xrd[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) xrd[i] = 256 * l32 + 16 * ((4 * kq + 2 * i + h) ^ (lane & 15));
    const uint32_t wrow = 144 * (64 * rq + l32);
    // qs bytes 8h..8h+7 of block jj start at byte 18jj + 2 + 8h of the row;
    // 18jj + 2 is 2 mod 4 for even jj and 0 mod 4 for odd jj (jj has the parity of kq).
    const uint32_t wsh = (kq & 1) ? 0u : 2u;
    const NibUnpack nib;
    const half2_t off_lo = {static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f)};
    const half2_t off_hi = {static_cast<half_t>(-72.0f), static_cast<half_t>(-72.0f)};

    struct Ops {
        half8_t xa[2][2];  // [k-step][token fragment]
        half8_t wb[2][2];  // [k-step][row fragment]
    };
    auto read_ops = [&](int u, Ops& o) {
        const uint8_t* xs = lds + (u % sk::kXRing) * kXSlot;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int ft = 0; ft < 2; ++ft)
                o.xa[i][ft] = *reinterpret_cast<const half8_t*>(xs + xrd[i] + 8192 * ft);
        const int jj = 4 * (u & 1) + kq;
        const uint8_t* ws = lds + kWOff + ((u >> 1) % sk::kWRing) * kWSlot + wrow;
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) {
            const uint8_t* rowp = ws + 4608 * fr;
            const uint16_t dbits = *reinterpret_cast<const uint16_t*>(rowp + 18 * jj);
            const uint32_t* qp = reinterpret_cast<const uint32_t*>(rowp + ((18 * jj + 2 + 8 * h) & ~3));
            const uint32_t d0 = qp[0], d1 = qp[1], d2 = wsh ? qp[2] : 0u;
            const uint32_t q0 = __builtin_amdgcn_alignbyte(d1, d0, wsh);
            const uint32_t q1 = __builtin_amdgcn_alignbyte(d2, d1, wsh);
            const half_t dv = __builtin_bit_cast(half_t, dbits);
            const half2_t dd = {dv, dv};
            const uint32_t t[4] = {__builtin_amdgcn_perm(0u, q0, 0x0C010C00u), __builtin_amdgcn_perm(0u, q0, 0x0C030C02u),
                                   __builtin_amdgcn_perm(0u, q1, 0x0C010C00u), __builtin_amdgcn_perm(0u, q1, 0x0C030C02u)};
            u32x4_t lo, hi;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                lo[e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, nib.lo_c(t[e])) + off_lo) * dd);
                hi[e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, nib.hi_c(t[e])) + off_hi) * dd);
            }
            o.wb[0][fr] = __builtin_bit_cast(half8_t, lo);
            o.wb[1][fr] = __builtin_bit_cast(half8_t, hi);
        }
    };

    float16_t acc[2][2];  // [token fragment][row fragment]
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][c][v] = 0.f;
    auto mma = [&](const Ops& o) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int ft = 0; ft < 2; ++ft)
#pragma unroll
                for (int fr = 0; fr < 2; ++fr)
                    acc[ft][fr] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o.xa[i][ft], o.wb[i][fr], acc[ft][fr], 0, 0, 0);
    };

    // ---- issue order (per wave): virtual stages -6 .. -1 issue what stages
    // s >= 0 issue at their top: X of stage s+4 (2 transfers), and on even s
    // super-block s/2+3 (3 transfers).  Before reading the operands of stage
    // u the wave waits for X(u): transfers issued after it number 7 for even
    // u-1 (the stage doing the wait) and 10 for odd; super-block u/2 went out
    // before X(u).
    issue_w(0);
    issue_x(0);
    issue_w(1);
    issue_x(1);
    issue_x(2);
    issue_w(2);
    issue_x(3);
    wait_vmcnt_asm<12>();  // X(0) and super-block 0 have landed
    lds_barrier();
    Ops cur, nxt;
    read_ops(0, cur);

    auto stage = [&](auto P_, int s) {
        constexpr int P = decltype(P_)::value;  // s & 1
        // operands of stage s+1 must have landed in every wave
        wait_vmcnt_asm<P == 0 ? 7 : 10>();
        lds_barrier();
        issue_x(s + 4);
        if constexpr (P == 0) issue_w((s >> 1) + 3);
        read_ops(s + 1, nxt);
        mma(cur);
        // Interleave: the operand reads first, then each MFMA of this stage
        // followed by a share of the next stage's dequantization, so the two
        // waves of a SIMD keep its VALU busy while the matrix core runs.
        __builtin_amdgcn_sched_group_barrier(0x100, 10, 0);  // LDS reads
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // eight VALU
        }
        cur = nxt;
    };
    for (int s = 0; s < nst; s += 2) {  // nst is even
        stage(std::integral_constant<int, 0>{}, s);
        stage(std::integral_constant<int, 1>{}, s + 1);
    }
    // no transfer into this workgroup's LDS may outlive it, and the
    // reduction below reuses the rings
    wait_vmcnt_asm<0>();
    lds_barrier();

    // ---- sum the four K-quarters of each output in kq order and store
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int ft = 0; ft < 2; ++ft)
#pragma unroll
        for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int idx = (wave * 16 + (ft * 2 + fr) * 4 + j) * 64 + lane;
                *reinterpret_cast<float4_t*>(red + 4 * idx) =
                    float4_t{acc[ft][fr][4 * j], acc[ft][fr][4 * j + 1], acc[ft][fr][4 * j + 2], acc[ft][fr][4 * j + 3]};
            }
    __syncthreads();
    // wave (kq, rq) stores fragment f = kq (token fragment kq >> 1, row fragment kq & 1) of row half rq
    {
        const int ft = kq >> 1, fr = kq & 1;
        const int m = m0 + 64 * rq + 32 * fr + l32;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float4_t sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int src = 0; src < 4; ++src) {
                const int idx = ((4 * rq + src) * 16 + kq * 4 + j) * 64 + lane;
                sum += *reinterpret_cast<const float4_t*>(red + 4 * idx);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + 32 * ft + 8 * j + 4 * h + i;
                if (t < T && m < M) Y[t * ldy + m] = f2h_bits(sum[i]);
            }
        }
    }
}

int launch_gemm_sk(const void* w, const void* x, void* y, int M, int K, int T, int64_t ldx, int64_t ldy,
                   hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(&dequant_gemm_q4_0_sk);
    if (int rc = prepare_lds(fn, sk::kLds)) return rc;
    const int64_t mtiles = (M + sk::kBM - 1) / sk::kBM;
    // one launch covers at most 2^30 workgroups; longer prompts take several
    constexpr int64_t kMaxWg = int64_t(1) << 30;
    const int64_t tchunk = std::max<int64_t>(1, kMaxWg / mtiles) * sk::kBT;
    for (int64_t t = 0; t < T; t += tchunk) {
        const int tc = static_cast<int>(std::min<int64_t>(T - t, tchunk));
        const unsigned nwg = static_cast<unsigned>(mtiles * ((tc + sk::kBT - 1) / sk::kBT));
        hipLaunchKernelGGL(dequant_gemm_q4_0_sk, dim3(nwg), dim3(sk::kWaves * 64), sk::kLds, stream,
                           static_cast<const uint8_t*>(w), static_cast<const uint16_t*>(x) + t * ldx,
                           static_cast<uint16_t*>(y) + t * ldy, M, K, tc, ldx, ldy, static_cast<int>(mtiles));
        if (int rc = check_hip(hipGetLastError(), "dequant_gemm_q4_0 launch")) return rc;
    }
    return GDSLLM_OK;
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
}  // namespace gdsllm

using namespace gdsllm;

extern "C" int gdsllm_dequant_gemm_q4_0(const void* weight, const void* x, void* y, int64_t out_dim, int64_t in_dim,
                                        int64_t tokens, int64_t ldx, int64_t ldy, void* stream) {
    const std::string n = "dequant_gemm_q4_0";
    if (out_dim < 0 || in_dim < 0 || tokens < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (in_dim % 32 != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": in_dim must be a multiple of 32, got " + std::to_string(in_dim));
    if (out_dim == 0 || in_dim == 0 || tokens == 0) return ok();
    if (!weight || !x || !y) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (ldx < in_dim || ldy < out_dim) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than the row length");
    if (out_dim > (int64_t(1) << 30) || in_dim > (int64_t(1) << 24) || tokens > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    if (reinterpret_cast<uintptr_t>(weight) % 16 || reinterpret_cast<uintptr_t>(x) % 16 || ldx % 8 ||
        reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": weight and x rows must be 16-byte aligned (ldx % 8 == 0)");
    // Wider token tiles dequantize each weight block fewer times, but a small
    // problem needs the narrower tiles to give every CU a workgroup: take the
    // widest tile (256, 128 or 64 tokens) that still does.
    const int M = static_cast<int>(out_dim), K = static_cast<int>(in_dim), T = static_cast<int>(tokens);
    const int64_t row_tiles = (M + kGemmRows - 1) / kGemmRows;
    auto tiles = [&](int bt) { return row_tiles * ((T + bt - 1) / bt); };
    const hipStream_t st = as_stream(stream);
    // the split-K kernel addresses X and W with 32-bit offsets inside a tile
    if (K % 256 == 0 && ldx <= (int64_t(1) << 24)) {
        const int rc = launch_gemm_sk(weight, x, y, M, K, T, ldx, ldy, st);
        return rc == GDSLLM_OK ? ok() : rc;
    }
    const int rc = tiles(256) >= cu_count()   ? launch_gemm<128>(weight, x, y, M, K, T, ldx, ldy, st)
                   : tiles(128) >= cu_count() ? launch_gemm<64>(weight, x, y, M, K, T, ldx, ldy, st)
                                              : launch_gemm<32>(weight, x, y, M, K, T, ldx, ldy, st);
    return rc == GDSLLM_OK ? ok() : rc;
}
