// Prefill dequant-GEMM for every weight format of the path, and the grouped
// expert GEMM of the MoE prefill, on the gfx950 matrix cores.
//
// Y[t][r] = fp16( sum_k X[t][k] * W[r][k] ) for a chunk of prompt tokens:
// what the reference's prefill branches compute as dequant -> F.linear
// (runtime/llama.py:160-166 for GGUF Q4_0 / Q8_0, runtime/qwen_moe.py:72-73
// for affine-Q4), fused so the fp16 weight matrix never goes back to HBM.
//
// One split-K workgroup kernel serves three weight formats and three modes.
//
// Workgroup: 128 weight rows x BT tokens (BT = 64 or 32), 8 waves (two per
// SIMD).  A stage is 128 values of k (four 32-value blocks); wave w takes
// block w & 3 of every stage for weight rows 64*(w >> 2) .. +63, so each
// weight is dequantized exactly once per workgroup, in registers, from its raw
// bytes in LDS.  The four K-quarters are summed through LDS at the end in a
// fixed order (results do not depend on timing).
//  * MFMA v_mfma_f32_32x32x16_f16, A = X (32 tokens x 16 k), B = W (16 k x 32
//    rows): lane l holds token/row l % 32 and k values 8(l/32) .. +7 of a
//    16-value k-step.
//  * Weight operands (fp16, into the matrix cores):
//      Q4_0  (q | 0x6400) - 1032 and (q<<4 | 0x5400) - 72 are q-8 exactly;
//            one packed multiply by d rounds once: the reference's
//            dequantized value (gguf_dequant.cu:105-106), bit for bit.
//      Q8_0  bytes xor 0x80 placed under an 0x64 exponent byte are 1024+q+128;
//            minus 1152 is q exactly; one packed multiply by d rounds once
//            (gguf_dequant.cu:52-57), bit for bit.
//      affine one byte's two nibbles become (1024+lo, 64+hi); minus (1024, 64)
//            is the nibble pair exactly; one packed fma with (s, b) rounds
//            nib*s+b once to fp16.  The reference rounds nib*s+b to fp32 first
//            (affine_q4_dequant.cu:50-58); the two differ only where that sum
//            is not exact in fp32, by one fp16 ulp of that weight.
//  * Data path: global -> LDS by DMA (global_load_lds), issued from inline
//    asm in the saddr form (wave-uniform base, fixed 32-bit lane offsets):
//    the compiler neither sees nor waits for the transfers, and its own LDS
//    operand reads are ordinary instructions scheduled between the MFMAs.
//    Every vector-memory operation in the main loop is one of these
//    transfers, so the vmcnt waits are exact compile-time counts.
//    X: ring of XR stage tiles; stage s issues X of stage s + XR into the
//    slot of stage s (read during stage s - 1, before this stage's barrier).
//    W: ring of RW slots, a slot holding SPS stages of 128 rows; the last
//    stage of group g issues group g + RW into the slot of group g.
//  * X tile layout: token t's 16 chunks of 16 bytes sit in one 256-byte row,
//    chunk c at position c ^ (t & 15): the lanes reading chunk c of 32
//    consecutive tokens hit distinct 16-byte bank groups.
//
// Modes:
//  * kDense   X rows t0 .. t0+BT-1, Y rows the same; workgroups are remapped
//             so that each XCD takes a contiguous, token-tile-major range of
//             tiles (its L2 keeps the X token tile while it streams weights).
//  * kGather  the tile list of the MoE prefill: tile (expert e, position p0,
//             count n) multiplies the X rows tok[p0 .. p0+n-1] by expert e's
//             matrix (stacked pool, e * stride) into Y rows p0 .. p0+n-1.
//  * kDenseDual kDense with the gate/up split of kDualSilu: workgroup rows
//             0..BM/2-1 from the gate matrix and BM/2..BM-1 from the up matrix
//             at the same BM/2 output rows, h written instead of g and u (the
//             prefill form of the decode gate_up_silu, runtime/llama.py:253-256).
//  * kDualSilu  kGather with rows 0..63 of the workgroup taken from the gate
//             pool and rows 64..127 from the up pool at the same 64 output
//             rows; the epilogue writes h = fp16(fp16(silu(g)) * u) with
//             torch's fp16 semantics (runtime/qwen_moe.py:488-490), so the
//             gate and up outputs never reach HBM.

#include <algorithm>

#include "common.h"

namespace gdsllm {
namespace {

enum class WF { Q4_0, Q8_0, AFF32, AFF64, AFF128 };
enum Mode { kDense = 0, kGather = 1, kDualSilu = 2, kDenseDual = 3 };

constexpr int kWaves = 8;
constexpr int kBM = 128;     // weight rows per workgroup (or 256: the dense tile of gemm_sk)
constexpr int kStageK = 128; // k values per stage

constexpr bool is_affine(WF f) { return f == WF::AFF32 || f == WF::AFF64 || f == WF::AFF128; }
constexpr int aff_group(WF f) { return f == WF::AFF32 ? 32 : f == WF::AFF64 ? 64 : 128; }

// W slot geometry per format.
//   SPS      stages per slot
//   kSlot    bytes of one slot (BM = 128 or 256 rows)
//   kReal    transfers that carry data per slot; kCW per wave (dummies past kReal)
//   GGUF: a 144-byte window per row (9 chunks): Q4_0 two stages (8 blocks of
//   18 bytes); Q8_0 one stage (4 blocks of 34 = 136 bytes, starting 0 or 8
//   bytes into the window).  Affine: 128 bytes of words per row (two stages),
//   then the rows' scales and biases for those 256 k values (SB bytes each).
template <WF F, int BM = kBM>
struct Fmt {
    static constexpr bool kAff = is_affine(F);
    static_assert(BM == kBM || BM == 2 * kBM, "128- or 256-row slots");
    static constexpr int G = kAff ? aff_group(F) : 32;
    static constexpr int SPS = F == WF::Q8_0 ? 1 : 2;
    static constexpr int SB = kAff ? 512 / G : 0;                          // scale bytes per row per slot
    static constexpr bool kS16 = SB == 16;                                 // scales move in 16-byte transfers
    static constexpr int kST = kAff ? (kS16 ? 2 * BM / kBM : SB * BM / 256) : 0;  // transfers for one of scales/biases
    static constexpr int kWords = 128 * BM;                                // affine: bytes of words per slot
    static constexpr int kSlot = kAff ? kWords + 2 * BM * SB : BM * 144;
    static constexpr int kReal = kAff ? kWords / 1024 + 2 * kST : BM * 144 / 1024;
    static constexpr int kCW = (kReal + kWaves - 1) / kWaves;              // transfers per wave per slot
    static_assert(kReal <= kCW * kWaves && kReal > (kCW - 1) * kWaves, "full rounds of transfers and a partial last");
};

// X and W rings.  The 256-row tile (36 KiB W slots) keeps two of each: a
// stage of it is two of a 128-row tile's stages long per wave, so two slots
// hide as much latency as three do there.  The 32-token tiles of the grouped
// MoE prefill keep 4 X and 2 W slots (69 KiB with affine g64), so two
// workgroups share a CU and one's pipeline fill and epilogue overlap the
// other's stream: each tile job is short (one expert's ~10 tokens), and with
// 6 + 5 slots (139 KiB, one workgroup per CU) the 512-token chunk over the
// 512-expert pool took 1560 us, with 4 + 2 slots 1178-1227 us.
template <WF F, int BT, int BM = kBM>
struct Ring {
    static constexpr int kXSlot = BT * 256;
    static constexpr int kLdsMax = 163840;
    static constexpr int XR0 = BM == 2 * kBM ? 2 : BT == 128 ? 3 : BT == 64 ? 5 : 4;
    static constexpr int RW = BM == 2 * kBM ? 2 : BT == 128 ? 3 : BT == 64 ? 4 : 2;
    static constexpr int XR = XR0 * kXSlot + RW * Fmt<F, BM>::kSlot + 1024 <= kLdsMax ? XR0 : XR0 - 1;
    static constexpr int kWOff = XR * kXSlot;
    static constexpr int kDummy = kWOff + RW * Fmt<F, BM>::kSlot;
    static constexpr int kRing = kDummy + 1024;  // dummy transfers land in the last 1 KiB
    static constexpr int kRed = kWaves * (BT >= 64 ? 2 : 1) * 2 * 4 * 64 * 16;  // partial sums of one pass
    static constexpr int kLds = kRing > kRed ? kRing : kRed;
    static_assert(kLds <= kLdsMax, "LDS budget");
};

// Transfers each wave has in flight after the one a stage waits for: the
// issue pattern repeats with period SPS (X every stage, NX per wave; W on the
// last stage of a group, CW per wave), so the count depends on s mod SPS only.
// Before reading the operands of stage s+1 (at the top of stage s, nothing of
// stage s issued yet) X(s+1) and W group (s+1)/SPS must have landed.
constexpr int stage_issues(int st, int SPS, int NX, int CW) { return NX + ((st % SPS == SPS - 1) ? CW : 0); }
constexpr int wait_count(int phase, int SPS, int XR, int RW, int NX, int CW) {
    const int s = 64 * SPS + phase;  // any stage with this phase, far from 0
    const int a = s + 1 - XR;        // X(s+1) goes out first in stage a
    int cx = (a % SPS == SPS - 1) ? CW : 0;
    for (int st = a + 1; st <= s - 1; ++st) cx += stage_issues(st, SPS, NX, CW);
    const int G = (s + 1) / SPS;
    const int b = (G - RW) * SPS + SPS - 1;  // W group G goes out last in stage b
    int cw = 0;
    for (int st = b + 1; st <= s - 1; ++st) cw += stage_issues(st, SPS, NX, CW);
    return cx < cw ? cx : cw;
}

struct GemmArgs {
    const uint8_t* w;   // GGUF blocks or affine words (dual mode: gate)
    const uint8_t* s;   // affine scales
    const uint8_t* b;   // affine biases
    const uint8_t* w2;  // dual mode: up
    const uint8_t* s2;
    const uint8_t* b2;
    int64_t estride_w, estride_s, estride_b;  // per-expert byte strides (gather modes)
    const uint16_t* x;
    uint16_t* y;
    int M, K, T;
    int64_t ldx, ldy;
    int mtiles;
    const int4* tiles;  // gather modes: (expert, p0, n, 0)
    const int* ntiles;
    const int* tok;     // gather modes: X row of each position
};

typedef float float16_t __attribute__((ext_vector_type(16)));

// BM = 256 (the dense modes): the same 64-row x BT-token wave tile, with
// the workgroup's 8 waves as 4 row quarters x 2 K halves instead of 2 row
// halves x 4 K quarters.  Each X stage then feeds twice the rows: per MFMA the
// compute unit takes in 40% fewer bytes (X dominates them), which is what
// bounds this kernel at 512 tokens.  A wave's stage is two sub-stages (its two
// blocks of the four), each scheduled like a 128-row stage; the wait and the
// workgroup barrier come once per stage, after the second.
template <WF F, int BT, int MODE, int BM = kBM>
__global__ __launch_bounds__(kWaves * 64) void gemm_sk(GemmArgs a) {
    using Fm = Fmt<F, BM>;
    using R = Ring<F, BT, BM>;
    constexpr int NTF = BT / 32;        // token fragments per wave
    constexpr int NX = BT / 32;         // X transfers per wave per stage
    constexpr int SPS = Fm::SPS, XR = R::XR, RW = R::RW, CW = Fm::kCW;
    constexpr int kXSlot = R::kXSlot;
    constexpr bool kGath = MODE == kGather || MODE == kDualSilu;
    constexpr bool kDual = MODE == kDualSilu || MODE == kDenseDual;
    static_assert(MODE != kDualSilu || Fm::kAff, "the gathered dual tiles are built for the affine pools");
    static_assert(BM == kBM || MODE == kDense || MODE == kDenseDual, "the 256-row tile serves the dense modes only");
    constexpr int KS = kWaves * 64 / BM;  // waves along K (4 or 2)
    constexpr int NSUB = 4 / KS;          // 32-value blocks per wave per stage

    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int kq = wave % KS, rq = wave / KS;

    // ---- tile
    int m0, t0 = 0, nt, p0 = 0;
    const uint8_t *wA = a.w, *sA = a.s, *bA = a.b, *wB = a.w2, *sB = a.s2, *bB = a.b2;
    if constexpr (kGath) {
        // The grid covers the worst case; the first ntiles * mtiles
        // workgroups take a job, in the XCD-aware order of the dense modes
        // over that count: an XCD takes a contiguous range of jobs, i.e. the
        // row tiles of the same experts, so an expert's token rows of X come
        // into one L2, not into all eight.
        const int jobs = __builtin_amdgcn_readfirstlane(*a.ntiles) * a.mtiles, b = blockIdx.x;
        if (b >= jobs) return;  // uniform
        const int per = jobs >> 3, rem = jobs & 7, xcd = b & 7;
        const int q = xcd * per + (xcd < rem ? xcd : rem) + (b >> 3);
        const int tile = q / a.mtiles;
        const int4 td = a.tiles[tile];
        m0 = (q % a.mtiles) * (kDual ? 64 : kBM);
        // wave-uniform values, said outright: the X issue branches on nt
        p0 = __builtin_amdgcn_readfirstlane(td.y);
        nt = __builtin_amdgcn_readfirstlane(td.z);
        const int64_t e = __builtin_amdgcn_readfirstlane(td.x);
        wA += e * a.estride_w;
        sA += e * a.estride_s;
        bA += e * a.estride_b;
        if constexpr (kDual) {
            wB += e * a.estride_w;
            sB += e * a.estride_s;
            bB += e * a.estride_b;
        }
    } else {
        // XCD-aware order: dispatch sends workgroup b to XCD b % 8
        const int nwg = gridDim.x, b = blockIdx.x;
        const int per = nwg >> 3, rem = nwg & 7, xcd = b & 7;
        const int q = xcd * per + (xcd < rem ? xcd : rem) + (b >> 3);
        m0 = (q % a.mtiles) * (kDual ? BM / 2 : BM);
        t0 = (q / a.mtiles) * BT;
        nt = min(BT, a.T - t0);
    }
    const int M = a.M, K = a.K;
    const int nst = K / kStageK, ngr = nst / SPS;
    const uint32_t lds0 = lds_addr(lds);

    // ---- X sources: transfer i of this wave (i = NX*wave + ii) fills 16-byte
    // slot 64i + l of a stage tile: token 4i + l/16, chunk (l & 15) ^ (token & 15).
    // Tokens past the tile read its last token.  The lane offsets are 32-bit:
    // the dense modes put the tile's first token into the 64-bit base (the
    // in-tile offsets stay below 2 * 128 * 2^24 bytes), the gathered modes
    // address whole rows of an X their entry point bounds below 4 GiB.
    uint32_t xoff[NX];
#pragma unroll
    for (int ii = 0; ii < NX; ++ii) {
        const int t = 4 * (NX * wave + ii) + (lane >> 4);
        const int c = (lane & 15) ^ (t & 15);
        const int tl = t < nt ? t : nt - 1;
        int64_t row;
        if constexpr (kGath) row = a.tok ? a.tok[p0 + tl] : p0 + tl;  // no list: X rows are the positions
        else row = tl;
        xoff[ii] = static_cast<uint32_t>(2 * (row * a.ldx + 8 * c));
    }
    const uint16_t* xbase = kGath ? a.x : a.x + static_cast<int64_t>(t0) * a.ldx;

    // ---- W sources.  Transfer i = 8*ii + wave of a slot (ii < CW: 3, or 5 for
    // the 256-row GGUF slot).  ii < CW - 1 are 16-byte transfers of GGUF
    // blocks / affine words (always data); ii = CW - 1 carries the last GGUF
    // transfers (16-17 of 18, 32-35 of 36), or the affine scales and biases,
    // and is a dummy in the remaining waves.  The kind of each ii is a
    // compile-time fact and its base and LDS offset are wave-uniform, so the
    // issue code has no branches; lane offsets are fixed per lane.
    const int64_t rb_main = Fm::kAff ? K / 2 : (K / 32) * (F == WF::Q8_0 ? 34 : 18);
    const int64_t rb_sc = Fm::kAff ? 2 * (K / Fm::G) : 0;
    constexpr bool k2s16 = !Fm::kAff || Fm::kS16;  // ii = CW - 1 moves 16 bytes per lane (else 4)
    constexpr int L = CW - 1;  // the last transfer of a slot, partly dummies
    // transfers per wave of GGUF blocks / affine words that are always data
    constexpr int NWI = Fm::kAff ? 2 * BM / kBM : L;
    const uint8_t* wsrc[CW];   // tile base (row m0 of its matrix)
    uint32_t woff[CW];
    uint32_t wdst[CW];         // LDS offset inside the slot
    bool real[CW];             // false: a dummy transfer
#pragma unroll
    for (int ii = 0; ii < NWI; ++ii) {
        const int i = 8 * ii + wave;
        int r, cp;
        if constexpr (!Fm::kAff) {
            const int g = 64 * i + lane;
            r = g / 9;
            cp = g % 9;
        } else {
            // chunk position p of row r holds the row's chunk p ^ (r & 7), so
            // the 32 rows a fragment reads at one word hit distinct banks
            const int g = 64 * i + lane;
            r = g >> 3;
            cp = (g & 7) ^ (r & 7);
        }
        const bool second = kDual && i >= (Fm::kAff ? 8 * NWI / 2 : Fm::kReal / 2);  // up rows BM/2 .. BM-1
        const int rr = second ? r - BM / 2 : r;
        const int ra = min(m0 + rr, M - 1) - m0;
        wsrc[ii] = (second ? wB : wA) + static_cast<int64_t>(m0) * rb_main;
        woff[ii] = static_cast<uint32_t>(ra * rb_main + 16 * cp);
        wdst[ii] = 1024 * i;
        real[ii] = true;
    }
    if constexpr (!Fm::kAff) {
        const int i = 8 * L + wave;
        real[L] = i < Fm::kReal;
        const int g = 64 * i + lane, r = g / 9, cp = g % 9;
        const bool second = kDual;  // rows past BM/2
        const int rr = second ? r - BM / 2 : r;
        const int ra = min(m0 + rr, M - 1) - m0;
        wsrc[L] = (second ? wB : wA) + static_cast<int64_t>(m0) * rb_main;
        woff[L] = real[L] ? static_cast<uint32_t>(ra * rb_main + 16 * cp) : 0u;
        wdst[L] = 1024 * i;
    } else {
        // scales then biases: transfer j0 = 8 (ii - NWI) + wave of the 2 kST
#pragma unroll
        for (int ii = NWI; ii < CW; ++ii) {
            const int j0 = 8 * (ii - NWI) + wave;
            real[ii] = j0 < 2 * Fm::kST;
            const bool isb = j0 >= Fm::kST;
            const int j = isb ? j0 - Fm::kST : j0;
            const bool second = kDual && j >= Fm::kST / 2;
            const uint8_t* base = isb ? (second ? bB : bA) : (second ? sB : sA);
            int r, inrow;
            if constexpr (Fm::kS16) {
                r = 64 * j + lane;
                inrow = 0;
                wdst[ii] = Fm::kWords + (isb ? BM * Fm::SB : 0) + 1024 * j;
            } else {
                const int d = 64 * j + lane, per = Fm::SB / 4;
                r = d / per;
                inrow = 4 * (d % per);
                wdst[ii] = Fm::kWords + (isb ? BM * Fm::SB : 0) + 256 * j;
            }
            const int rr = second ? r - BM / 2 : r;
            const int ra = min(m0 + rr, M - 1) - m0;
            wsrc[ii] = (real[ii] ? base : sA) + static_cast<int64_t>(m0) * rb_sc;
            woff[ii] = real[ii] ? static_cast<uint32_t>(ra * rb_sc + inrow) : 0u;
        }
    }
    // byte offset of group gi inside a row: GGUF blocks / affine words
    auto goff_main = [&](int gi) -> int64_t {
        if constexpr (F == WF::Q4_0) return 144 * static_cast<int64_t>(gi);
        else if constexpr (F == WF::Q8_0) return 136 * static_cast<int64_t>(gi) - 8 * (gi & 1);
        else return 128 * static_cast<int64_t>(gi);
    };

    // Gathered tiles: a transfer whose four tokens all lie past the tile's
    // count (an expert's ~10 tokens in a 32-token tile) is a dummy, so the
    // compute unit takes in only the token rows that exist.  Their slot rows
    // keep older data; they feed only the MFMA outputs of those tokens, which
    // are never stored.
    bool xlive[NX];
#pragma unroll
    for (int ii = 0; ii < NX; ++ii) xlive[ii] = !kGath || 4 * (NX * wave + ii) < nt;
    auto issue_x = [&](int sx) {  // X of stage sx (any integer) into its ring slot
        const int sl = ((sx % XR) + XR) % XR;
        const uint32_t dst = lds0 + sl * kXSlot + 1024 * (NX * wave);
        if (sx < 0) {
#pragma unroll
            for (int ii = 0; ii < NX; ++ii) dma4_asm(0u, a.w, lds0 + R::kDummy);
            return;
        }
        const uint16_t* base = xbase + kStageK * (sx < nst ? sx : nst - 1);
#pragma unroll
        for (int ii = 0; ii < NX; ++ii) {
            if (xlive[ii]) dma16_asm(xoff[ii], base, dst + 1024 * ii);
            else dma4_asm(0u, a.w, lds0 + R::kDummy);
        }
    };
    auto issue_w = [&](int gi) {  // W group gi into its ring slot
        if (gi < 0) {
#pragma unroll
            for (int ii = 0; ii < CW; ++ii) dma4_asm(0u, a.w, lds0 + R::kDummy);
            return;
        }
        const uint32_t slot = lds0 + R::kWOff + (gi % RW) * Fm::kSlot;
        const int gc = gi < ngr ? gi : ngr - 1;
        const int64_t om = goff_main(gc);
#pragma unroll
        for (int ii = 0; ii < NWI; ++ii) dma16_asm(woff[ii], wsrc[ii] + om, slot + wdst[ii]);
        const int64_t o2 = Fm::kAff ? static_cast<int64_t>(Fm::SB) * gc : om;
#pragma unroll
        for (int ii = NWI; ii < CW; ++ii) {
            const uint32_t d2 = real[ii] ? slot + wdst[ii] : lds0 + R::kDummy;
            if constexpr (k2s16) dma16_asm(woff[ii], wsrc[ii] + o2, d2);
            else dma4_asm(woff[ii], wsrc[ii] + o2, d2);
        }
    };
    auto floordiv = [](int v, int d) { return v >= 0 ? v / d : -((-v + d - 1) / d); };
    auto issue_stage = [&](int s) {
        issue_x(s + XR);
        const int ph = ((s % SPS) + SPS) % SPS;
        if (ph == SPS - 1) issue_w(floordiv(s, SPS) + RW);
    };

    // ---- operand reads of sub-stage j of stage u: block NSUB*kq + j of the stage
    uint32_t xrd[NSUB][2];
#pragma unroll
    for (int j = 0; j < NSUB; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i) xrd[j][i] = 256 * l32 + 16 * ((4 * (NSUB * kq + j) + 2 * i + h) ^ (lane & 15));
    const int row0 = 64 * rq + l32;  // tile row of fragment 0
    // qs bytes 8h.. of a block start 2 mod 4 bytes into LDS for even blocks
    auto wshift = [&](int j) -> uint32_t { return ((NSUB * kq + j) & 1) ? 0u : 2u; };
    const NibUnpack nib;
    uint32_t c64 = 0x64646464u, mixmask = 0x00F0000Fu, mixbits = 0x54006400u;
    asm volatile("" : "+v"(c64), "+s"(mixmask), "+v"(mixbits));
    const half2_t off_lo = {static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f)};
    const half2_t off_hi = {static_cast<half_t>(-72.0f), static_cast<half_t>(-72.0f)};
    const half2_t off_q8 = {static_cast<half_t>(-1152.0f), static_cast<half_t>(-1152.0f)};
    const half2_t off_mix = {static_cast<half_t>(-1024.0f), static_cast<half_t>(-64.0f)};

    // Operands of one stage: X fragments straight from LDS, weight fragments
    // dequantized in eight units (two row fragments x four) from raw LDS words.
    struct Raw {
        half8_t xa[2][NTF];  // [k-step][token fragment]
        uint32_t q[2][6];    // [row fragment] raw dwords (GGUF: 3 per k-step group; affine: 2 words)
        uint16_t d[2][2];    // [row fragment] GGUF scale bits / affine scale, bias bits
    };
    struct Wb {
        u32x4_t v[2][2];     // [k-step][row fragment]: fp16 weight pairs
        uint32_t t[2][4];    // [row fragment] prepared bytes shared by a fragment's units
    };
    auto read_raw = [&](int u, int j, Raw& o) {
        const int kb = NSUB * kq + j;  // block of the stage
        const uint8_t* xs = lds + (u % XR) * kXSlot;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int ft = 0; ft < NTF; ++ft)
                o.xa[i][ft] = *reinterpret_cast<const half8_t*>(xs + xrd[j][i] + 8192 * ft);
        const uint8_t* ws = lds + R::kWOff + ((u / SPS) % RW) * Fm::kSlot;
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) {
            const int rt = row0 + 32 * fr;
            // a block's qs bytes 8h.. (k-step pairs) are read as whole dwords; the
            // third dword is read even when unused (inside the slot, or the bytes
            // after the ring), so no branch splits the loop body
            if constexpr (F == WF::Q4_0) {
                const int jj = 4 * (u & 1) + kb;
                const uint8_t* rowp = ws + 144 * rt;
                o.d[fr][0] = *reinterpret_cast<const uint16_t*>(rowp + 18 * jj);
                const uint32_t* qp = reinterpret_cast<const uint32_t*>(rowp + ((18 * jj + 2 + 8 * h) & ~3));
                o.q[fr][0] = qp[0];
                o.q[fr][1] = qp[1];
                o.q[fr][2] = qp[2];
            } else if constexpr (F == WF::Q8_0) {
                const int blk = 8 * (u & 1) + 34 * kb;
                const uint8_t* rowp = ws + 144 * rt;
                o.d[fr][0] = *reinterpret_cast<const uint16_t*>(rowp + blk);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t* qp = reinterpret_cast<const uint32_t*>(rowp + ((blk + 2 + 16 * i + 8 * h) & ~3));
                    o.q[fr][3 * i] = qp[0];
                    o.q[fr][3 * i + 1] = qp[1];
                    o.q[fr][3 * i + 2] = qp[2];
                }
            } else {
                // words 16(u & 1) + 4kb + 2i + h of the row: chunk 4(u & 1) + kb
                const uint8_t* chunk = ws + 128 * rt + 16 * ((4 * (u & 1) + kb) ^ (rt & 7));
                o.q[fr][0] = *reinterpret_cast<const uint32_t*>(chunk + 4 * h);
                o.q[fr][1] = *reinterpret_cast<const uint32_t*>(chunk + 4 * h + 8);
                const int gi = (128 * (u & 1) + 32 * kb) / Fm::G;
                const uint8_t* sp = ws + Fm::kWords + Fm::SB * rt + 2 * gi;
                o.d[fr][0] = *reinterpret_cast<const uint16_t*>(sp);
                o.d[fr][1] = *reinterpret_cast<const uint16_t*>(sp + BM * Fm::SB);
            }
        }
    };
    // Dequant unit (ks, z) of the weight fragments: k-step ks, row fragment
    // z / 2, pairs 2(z & 1) .. +1 of the fragment's four.  A k-step's four units
    // run in order (unit 0 of a fragment prepares the bytes its units share).
    auto dq_unit = [&](int ks, int z, const Raw& r, Wb& o, uint32_t wsh) {
        const int fr = z >> 1, hf = z & 1;
        if constexpr (F == WF::Q4_0) {
            // k-step 0 takes the low nibbles, k-step 1 the high nibbles of the same bytes
            if (ks == 0 && hf == 0) {
                const uint32_t q0 = __builtin_amdgcn_alignbyte(r.q[fr][1], r.q[fr][0], wsh);
                const uint32_t q1 = __builtin_amdgcn_alignbyte(r.q[fr][2], r.q[fr][1], wsh);
                o.t[fr][0] = __builtin_amdgcn_perm(0u, q0, 0x0C010C00u);
                o.t[fr][1] = __builtin_amdgcn_perm(0u, q0, 0x0C030C02u);
                o.t[fr][2] = __builtin_amdgcn_perm(0u, q1, 0x0C010C00u);
                o.t[fr][3] = __builtin_amdgcn_perm(0u, q1, 0x0C030C02u);
            }
            const half_t dv = __builtin_bit_cast(half_t, r.d[fr][0]);
            const half2_t dd = {dv, dv};
#pragma unroll
            for (int e = 2 * hf; e < 2 * hf + 2; ++e) {
                if (ks == 0)
                    o.v[0][fr][e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, nib.lo_c(o.t[fr][e])) + off_lo) * dd);
                else
                    o.v[1][fr][e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, nib.hi_c(o.t[fr][e])) + off_hi) * dd);
            }
        } else if constexpr (F == WF::Q8_0) {
            if (hf == 0) {
                o.t[fr][2 * ks] = __builtin_amdgcn_alignbyte(r.q[fr][3 * ks + 1], r.q[fr][3 * ks], wsh) ^ 0x80808080u;
                o.t[fr][2 * ks + 1] = __builtin_amdgcn_alignbyte(r.q[fr][3 * ks + 2], r.q[fr][3 * ks + 1], wsh) ^ 0x80808080u;
            }
            const half_t dv = __builtin_bit_cast(half_t, r.d[fr][0]);
            const half2_t dd = {dv, dv};
            const uint32_t v = o.t[fr][2 * ks + hf];
            const uint32_t p0 = __builtin_amdgcn_perm(c64, v, 0x04010400u), p1 = __builtin_amdgcn_perm(c64, v, 0x04030402u);
            o.v[ks][fr][2 * hf] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, p0) + off_q8) * dd);
            o.v[ks][fr][2 * hf + 1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, p1) + off_q8) * dd);
        } else {
            const half_t sv = __builtin_bit_cast(half_t, r.d[fr][0]), bv = __builtin_bit_cast(half_t, r.d[fr][1]);
            const half2_t ss = {sv, sv}, bb = {bv, bv};
#pragma unroll
            for (int e = 2 * hf; e < 2 * hf + 2; ++e) {
                const uint32_t t = __builtin_amdgcn_perm(0u, r.q[fr][ks], 0x0C000C00u | (0x00010001u * e));
                const half2_t pr = __builtin_bit_cast(half2_t, (t & mixmask) | mixbits) + off_mix;  // exact nibbles
                o.v[ks][fr][e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(pr, ss, bb));
            }
        }
    };

    float16_t acc[NTF][2];  // [token fragment][row fragment]
#pragma unroll
    for (int ft = 0; ft < NTF; ++ft)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[ft][c][v] = 0.f;
    // MFMA z of a stage: k-step i = z / (2 NTF), then token fragment, then row
    // fragment; the two k-steps of one accumulator are 2 NTF MFMAs apart
    auto mfma_z = [&](int z, const Raw& r, const Wb& w) {
        const int i = z / (2 * NTF), ft = (z / 2) % NTF, fr = z & 1;
        acc[ft][fr] = __builtin_amdgcn_mfma_f32_32x32x16_f16(r.xa[i][ft], __builtin_bit_cast(half8_t, w.v[i][fr]),
                                                             acc[ft][fr], 0, 0, 0);
    };

    // ---- prologue: the issue pattern of stages -P .. -1 (dummies where a
    // stage would issue before stage 0's data), so the counts stay periodic
    constexpr int P = XR > (RW - 1) * SPS + 1 ? XR : (RW - 1) * SPS + 1;
    for (int s = -P; s < 0; ++s) issue_stage(s);
    wait_vmcnt_asm<wait_count(SPS - 1, SPS, XR, RW, NX, CW)>();
    lds_barrier();
    Raw rcur, rnxt;
    Wb wcur, wnxt;
    read_raw(0, 0, rcur);
#pragma unroll
    for (int z = 0; z < 4; ++z) dq_unit(0, z, rcur, wcur, wshift(0));

    // A stage in two halves, one per k-step of its MFMAs:
    //  1. the k-step 0 MFMAs of stage s (operands already in registers), with
    //     the k-step 1 weights of stage s dequantized between them;
    //  2. the wait for the landed bundle, the workgroup barrier, the next
    //     transfers and the raw operand reads of stage s+1;
    //  3. the k-step 1 MFMAs of stage s, with the k-step 0 weights of stage
    //     s+1 dequantized between them after the first Z0 (which cover the
    //     LDS read latency).
    // The matrix core thus runs through the barrier and the transfer issue,
    // and the dequant VALU is spread over all MFMAs.  Scheduling barriers keep
    // this order: left alone, the compiler groups all VALU and all MFMAs.
    constexpr int NH = 2 * NTF;          // MFMAs per k-step
    constexpr int Z0 = NH >= 8 ? 3 : 1;  // k-step 1 MFMAs before the first unit of stage s+1
    auto spread = [&](int z, int zfirst, int nz, auto&& unit) {
        // units u with (u * nz) / 4 == z - zfirst, i.e. 4 units over nz slots
        if (z < zfirst) return;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if ((u * nz) / 4 == z - zfirst) unit(u);
    };
    // Sub-stage J of stage s.  Only the last one waits, meets the workgroup
    // at the barrier and issues transfers; an earlier one reads the next
    // block of the same stage, which landed before the previous barrier.
    auto sub_stage = [&](auto P_, auto J_, int s) {
        constexpr int PH = decltype(P_)::value;  // s % SPS
        constexpr int J = decltype(J_)::value;
        const uint32_t sh_cur = wshift(J), sh_nxt = wshift(J + 1 < NSUB ? J + 1 : 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int z = 0; z < NH; ++z) {
            mfma_z(z, rcur, wcur);
            spread(z, 0, NH, [&](int u) { dq_unit(1, u, rcur, wcur, sh_cur); });
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (J == NSUB - 1) {
            wait_vmcnt_asm<wait_count(PH, SPS, XR, RW, NX, CW)>();
            lds_barrier();
            issue_x(s + XR);
            if constexpr (PH == SPS - 1) issue_w(s / SPS + RW);
            read_raw(s + 1, 0, rnxt);
        } else {
            read_raw(s, J + 1, rnxt);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int z = NH; z < 2 * NH; ++z) {
            mfma_z(z, rcur, wcur);
            spread(z - NH, Z0, NH - Z0, [&](int u) { dq_unit(0, u, rnxt, wnxt, sh_nxt); });
            __builtin_amdgcn_sched_barrier(0);
        }
        rcur = rnxt;
        wcur.v[0][0] = wnxt.v[0][0];
        wcur.v[0][1] = wnxt.v[0][1];
#pragma unroll
        for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int e = 0; e < 4; ++e) wcur.t[fr][e] = wnxt.t[fr][e];
    };
    auto stage = [&](auto P_, int s) {
        sub_stage(P_, std::integral_constant<int, 0>{}, s);
        if constexpr (NSUB == 2) sub_stage(P_, std::integral_constant<int, 1>{}, s);
    };
    if constexpr (SPS == 2) {
        for (int s = 0; s < nst; s += 2) {
            stage(std::integral_constant<int, 0>{}, s);
            stage(std::integral_constant<int, 1>{}, s + 1);
        }
    } else {
        for (int s = 0; s < nst; ++s) stage(std::integral_constant<int, 0>{}, s);
    }
    // no transfer into this workgroup's LDS may outlive it, and the
    // reduction below reuses the rings
    wait_vmcnt_asm<0>();
    lds_barrier();

    // ---- partial sums, in passes of PF token fragments (the LDS holds the
    // partials of two fragments per wave): unit (wave, f, fr, j) = 4 fp32
    // values per lane, tokens 32(pass*PF + f) + 8j + 4h + i (i < 4), tile row
    // 64rq + 32fr + l32
    constexpr int PF = NTF < 2 ? NTF : 2;
    float* red = reinterpret_cast<float*>(lds);
    auto unit = [&](int w, int f, int fr, int j) { return ((w * PF + f) * 2 + fr) * 4 + j; };
    auto ksum = [&](int wbase, int f, int fr, int j) {
        float4_t sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int src = 0; src < KS; ++src) sum += *reinterpret_cast<const float4_t*>(red + 4 * (unit(wbase + src, f, fr, j) * 64 + lane));
        return sum;
    };
    auto yrow = [&](int t) -> int64_t { return kGath ? static_cast<int64_t>(p0 + t) : static_cast<int64_t>(t0 + t); };
#pragma unroll
    for (int pass = 0; pass < NTF / PF; ++pass) {
        if (pass > 0) __syncthreads();  // the previous pass has read its partials
#pragma unroll
        for (int f = 0; f < PF; ++f)
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float16_t& av = acc[pass * PF + f][fr];
                    *reinterpret_cast<float4_t*>(red + 4 * (unit(wave, f, fr, j) * 64 + lane)) =
                        float4_t{av[4 * j], av[4 * j + 1], av[4 * j + 2], av[4 * j + 3]};
                }
        __syncthreads();
        if constexpr (!kDual) {
            // wave (kq, rq) stores units v = UPW*kq .. +UPW-1 of row block rq
            constexpr int UPW = 8 * PF / KS;
#pragma unroll
            for (int z = 0; z < UPW; ++z) {
                const int v = UPW * kq + z;
                const int j = v & 3, fr = (v >> 2) & 1, f = v >> 3;
                const float4_t sum = ksum(KS * rq, f, fr, j);
                const int m = m0 + 64 * rq + 32 * fr + l32;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 32 * (pass * PF + f) + 8 * j + 4 * h + i;
                    if (t < nt && m < M) a.y[yrow(t) * a.ldy + m] = f2h_bits(sum[i]);
                }
            }
        } else {
            // BM/2 output rows in GB 64-row blocks: wave w takes units
            // UD*w .. of the gate half, pairing each gate sum (row block gb,
            // waves KS*gb ..) with the up sum of row block gb + GB
            constexpr int GB = BM / 128, UD = GB * PF;
#pragma unroll
            for (int z = 0; z < UD; ++z) {
                const int va = UD * wave + z, gb = va / (8 * PF), v = va % (8 * PF);
                const int j = v & 3, fr = (v >> 2) & 1, f = v >> 3;
                const float4_t gs = ksum(KS * gb, f, fr, j), us = ksum(KS * (gb + GB), f, fr, j);
                const int m = m0 + 64 * gb + 32 * fr + l32;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 32 * (pass * PF + f) + 8 * j + 4 * h + i;
                    if (t < nt && m < M) a.y[yrow(t) * a.ldy + m] = silu_mul_h(gs[i], us[i]);
                }
            }
        }
    }
}

template <WF F, int BT, int MODE, int BM = kBM>
int launch_sk(const GemmArgs& a, unsigned nwg, hipStream_t stream) {
    using R = Ring<F, BT, BM>;
    const void* fn = reinterpret_cast<const void*>(&gemm_sk<F, BT, MODE, BM>);
    if (int rc = prepare_lds(fn, R::kLds)) return rc;
    hipLaunchKernelGGL((gemm_sk<F, BT, MODE, BM>), dim3(nwg), dim3(kWaves * 64), R::kLds, stream, a);
    return check_hip(hipGetLastError(), "prefill gemm launch");
}

// Dense GEMM over token chunks of at most 2^30 / mtiles tiles per launch.
template <WF F, int BT, int BM = kBM>
int dense_gemm(GemmArgs a, hipStream_t stream) {
    const int64_t mtiles = (a.M + BM - 1) / BM;
    a.mtiles = static_cast<int>(mtiles);
    const int64_t tchunk = std::max<int64_t>(1, (int64_t(1) << 30) / mtiles) * BT;
    const int T = a.T;
    const uint16_t* x0 = a.x;
    uint16_t* y0 = a.y;
    for (int64_t t = 0; t < T; t += tchunk) {
        const int tc = static_cast<int>(std::min<int64_t>(T - t, tchunk));
        a.x = x0 + t * a.ldx;
        a.y = y0 + t * a.ldy;
        a.T = tc;
        const unsigned nwg = static_cast<unsigned>(mtiles * ((tc + BT - 1) / BT));
        if (int rc = launch_sk<F, BT, kDense, BM>(a, nwg, stream)) return rc;
    }
    return GDSLLM_OK;
}

// Tile shape of a dense launch: the one with the least estimated time,
// rounds of the CUs (tile jobs / CUs, rounded up) times the time of one tile
// job, about 9 us of fixed cost (launch, pipeline fill, the K-part reduction)
// plus 24 us x r per 4096 of K, r = 1.1 for 128 rows x 64 tokens, 1.7 for
// 128 x 128 (the same dequant, twice the MFMAs) and 2.6 for 256 x 128 (twice
// the dequant and the MFMAs, X shared by twice the rows): fitted to Q4_0 tile
// jobs on MI355X (one round at K = 4096: 31-37, 51 and 69-75 us).  Ties take
// the smaller tile.  So 512 tokens over 11008 rows take 256 x 128 (1 round
// against 2 of 128 x 128 and 3 of 128 x 64), 256 tokens over 11008 rows and
// 128 tokens over 28672 or 32000 rows take 128 x 128 (1 round against 2),
// 512 tokens over 4096 rows 128 x 64.
enum class Tile { k128x64, k128x128, k256x128 };
inline Tile pick_tile(int64_t rows, int64_t T, int64_t K, bool allow256) {
    const int64_t cu = cu_count();
    auto rounds = [&](int64_t bm, int64_t bt) {
        return static_cast<double>(((rows + bm - 1) / bm * ((T + bt - 1) / bt) + cu - 1) / cu);
    };
    const double unit = 24.0 * static_cast<double>(K) / 4096.0;
    const double c64 = rounds(128, 64) * (9.0 + 1.1 * unit), c128 = rounds(128, 128) * (9.0 + 1.7 * unit),
                 c256 = rounds(256, 128) * (9.0 + 2.6 * unit);
    if (allow256 && c256 < c128 && c256 < c64) return Tile::k256x128;
    return c128 < c64 ? Tile::k128x128 : Tile::k128x64;
}

template <WF F>
int dense_gemm_auto(const GemmArgs& a, hipStream_t stream) {
    switch (pick_tile(a.M, a.T, a.K, true)) {
        case Tile::k256x128: return dense_gemm<F, 128, 2 * kBM>(a, stream);
        case Tile::k128x128: return dense_gemm<F, 128>(a, stream);
        default: return dense_gemm<F, 64>(a, stream);
    }
}

// Gate/up/SiLU over token chunks: BM/2 output rows per workgroup (gate rows in
// one half, up rows in the other), the 128-token tile when it fills every CU.
template <WF F, int BT, int BM = kBM>
int dense_dual_gemm(GemmArgs a, hipStream_t stream) {
    const int64_t mtiles = (a.M + BM / 2 - 1) / (BM / 2);
    a.mtiles = static_cast<int>(mtiles);
    const int64_t tchunk = std::max<int64_t>(1, (int64_t(1) << 30) / mtiles) * BT;
    const int T = a.T;
    const uint16_t* x0 = a.x;
    uint16_t* y0 = a.y;
    for (int64_t t = 0; t < T; t += tchunk) {
        const int tc = static_cast<int>(std::min<int64_t>(T - t, tchunk));
        a.x = x0 + t * a.ldx;
        a.y = y0 + t * a.ldy;
        a.T = tc;
        const unsigned nwg = static_cast<unsigned>(mtiles * ((tc + BT - 1) / BT));
        if (int rc = launch_sk<F, BT, kDenseDual, BM>(a, nwg, stream)) return rc;
    }
    return GDSLLM_OK;
}

// The tile shape as for the dense GEMM over the 2M gate and up rows (half
// of a tile's rows from each), 256-row tiles only where they halve the
// rounds of 128 x 128 ones (the 22016 rows of the LLaMA-7B gate/up/SiLU
// launch at 512 tokens, 2 rounds against 3, measured 138.9 against 134.8 us
// with 128-row tiles); affine weights keep 128-row tiles.
template <WF F>
int dense_dual_gemm_auto(const GemmArgs& a, hipStream_t stream) {
    const int64_t rows = 2 * static_cast<int64_t>(a.M), cu = cu_count();
    const int64_t r128 = ((rows + 127) / 128 * ((a.T + 127) / 128) + cu - 1) / cu;
    const int64_t r256 = ((rows + 255) / 256 * ((a.T + 127) / 128) + cu - 1) / cu;
    switch (pick_tile(rows, a.T, a.K, !is_affine(F) && 2 * r256 <= r128)) {
        case Tile::k256x128:
            if constexpr (!is_affine(F)) return dense_dual_gemm<F, 128, 2 * kBM>(a, stream);
            return dense_dual_gemm<F, 128>(a, stream);
        case Tile::k128x128: return dense_dual_gemm<F, 128>(a, stream);
        default: return dense_dual_gemm<F, 64>(a, stream);
    }
}

// ------------------------------------------------------------ MoE prefill --
//
// moe_sort (one workgroup): the T*k routed (token, slot) entries sorted by
// expert.  tok[p] is the token of position p, pos[t*k + j] the position of
// entry (t, j) (-1 for an expert index outside [0, E)), tiles[] the
// (expert, p0, n) token tiles of at most BT positions, *ntiles their count.
// The order of positions inside one expert is not fixed (LDS atomics); each
// output row depends only on its own token and expert, so results are.
constexpr int kSortThreads = 1024;
constexpr int kSortMaxExperts = 4096;

__global__ __launch_bounds__(kSortThreads) void moe_sort(const int32_t* __restrict__ idx, int n_entries, int top_k,
                                                         int E, int BT, int* __restrict__ tok, int* __restrict__ pos,
                                                         int4* __restrict__ tiles, int* __restrict__ ntiles) {
    __shared__ int cnt[kSortMaxExperts], off[kSortMaxExperts], toff[kSortMaxExperts];
    __shared__ int part[kSortThreads], tpart[kSortThreads];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += kSortThreads) cnt[e] = 0;
    __syncthreads();
    for (int i = tid; i < n_entries; i += kSortThreads) {
        const int e = idx[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive scans of the counts and of the tile counts: each thread sums a
    // contiguous run of experts, then a scan over the threads
    const int per = (E + kSortThreads - 1) / kSortThreads;
    const int e0 = min(E, tid * per), e1 = min(E, e0 + per);
    int sc = 0, st = 0;
    for (int e = e0; e < e1; ++e) {
        sc += cnt[e];
        st += (cnt[e] + BT - 1) / BT;
    }
    part[tid] = sc;
    tpart[tid] = st;
    __syncthreads();
    for (int d = 1; d < kSortThreads; d <<= 1) {
        const int pc = tid >= d ? part[tid - d] : 0, pt = tid >= d ? tpart[tid - d] : 0;
        __syncthreads();
        part[tid] += pc;
        tpart[tid] += pt;
        __syncthreads();
    }
    int rc = part[tid] - sc, rt = tpart[tid] - st;
    for (int e = e0; e < e1; ++e) {
        off[e] = rc;
        toff[e] = rt;
        rc += cnt[e];
        rt += (cnt[e] + BT - 1) / BT;
    }
    if (tid == kSortThreads - 1) *ntiles = tpart[tid];
    __syncthreads();
    for (int e = tid; e < E; e += kSortThreads) {
        const int c = cnt[e], o = off[e];
        for (int j = 0; j * BT < c; ++j) tiles[toff[e] + j] = int4{e, o + j * BT, min(BT, c - j * BT), 0};
        cnt[e] = 0;  // reused as the fill cursor
    }
    __syncthreads();
    for (int i = tid; i < n_entries; i += kSortThreads) {
        const int e = idx[i];
        if (e >= 0 && e < E) {
            const int p = off[e] + atomicAdd(&cnt[e], 1);
            tok[p] = i / top_k;
            pos[i] = p;
        } else {
            pos[i] = -1;
        }
    }
}

// expert_output of the prefill branch (runtime/qwen_moe.py:475-492) from the
// per-position down outputs: for each token, in slot order j = 0 .. k-1,
// acc = fp16(acc + fp16(w[t][j] * D[pos[t][j]])) with fp16 tensor semantics
// (each product and sum computed in fp32 and rounded to fp16).  Thread per 8
// columns of one token.
__global__ __launch_bounds__(256) void moe_prefill_combine(const uint16_t* __restrict__ D, const int* __restrict__ pos,
                                                           const uint16_t* __restrict__ w, int top_k, int H, int T,
                                                           uint16_t* __restrict__ y, int64_t ldy) {
    const int cpr = H / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(T) * cpr) return;
    const int t = static_cast<int>(i / cpr), c8 = static_cast<int>(i % cpr) * 8;
    float acc[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) acc[v] = 0.f;
    for (int j = 0; j < top_k; ++j) {
        const int p = pos[t * top_k + j];
        if (p < 0) continue;
        const float wk = h2f(w[t * top_k + j]);
        const uint4 d = *reinterpret_cast<const uint4*>(D + static_cast<int64_t>(p) * H + c8);
        const uint32_t dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float prod = h2f(f2h_bits(fp32_rounded(wk * h2f(dv[v >> 1] >> (16 * (v & 1))))));
            acc[v] = h2f(f2h_bits(fp32_rounded(acc[v] + prod)));
        }
    }
    uint4 o;
    o.x = static_cast<uint32_t>(f2h_bits(acc[0])) | (static_cast<uint32_t>(f2h_bits(acc[1])) << 16);
    o.y = static_cast<uint32_t>(f2h_bits(acc[2])) | (static_cast<uint32_t>(f2h_bits(acc[3])) << 16);
    o.z = static_cast<uint32_t>(f2h_bits(acc[4])) | (static_cast<uint32_t>(f2h_bits(acc[5])) << 16);
    o.w = static_cast<uint32_t>(f2h_bits(acc[6])) | (static_cast<uint32_t>(f2h_bits(acc[7])) << 16);
    *reinterpret_cast<uint4*>(y + static_cast<int64_t>(t) * ldy + c8) = o;
}

constexpr int kMoeBT = 32;

struct PrefillLayout {
    size_t tok, pos, tiles, ntiles, h, d, total;
};
PrefillLayout prefill_layout(int64_t T, int64_t k, int64_t F, int64_t H, int64_t E) {
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    const int64_t n = T * k;
    const int64_t max_tiles = n / kMoeBT + std::min<int64_t>(E, n) + 1;
    PrefillLayout L;
    size_t o = 0;
    L.tok = o;
    o = up(o + 4 * n);
    L.pos = o;
    o = up(o + 4 * n);
    L.tiles = o;
    o = up(o + 16 * max_tiles);
    L.ntiles = o;
    o = up(o + 16);
    L.h = o;
    o = up(o + 2 * n * F);
    L.d = o;
    o = up(o + 2 * n * H);
    L.total = o;
    return L;
}

template <WF F>
int moe_prefill_run(const gdsllm_affine_experts& g, const gdsllm_affine_experts& u, const gdsllm_affine_experts& d,
                    const void* x, int64_t ldx, const int32_t* idx, const void* rw, int64_t T, int64_t k, void* y,
                    int64_t ldy, uint8_t* ws, hipStream_t stream) {
    const int64_t E = g.num_experts, H = g.in_dim, Fd = g.out_dim, n = T * k;
    const PrefillLayout L = prefill_layout(T, k, Fd, H, E);
    int* tok = reinterpret_cast<int*>(ws + L.tok);
    int* pos = reinterpret_cast<int*>(ws + L.pos);
    int4* tiles = reinterpret_cast<int4*>(ws + L.tiles);
    int* ntiles = reinterpret_cast<int*>(ws + L.ntiles);
    uint16_t* hbuf = reinterpret_cast<uint16_t*>(ws + L.h);
    uint16_t* dbuf = reinterpret_cast<uint16_t*>(ws + L.d);
    hipLaunchKernelGGL(moe_sort, dim3(1), dim3(kSortThreads), 0, stream, idx, static_cast<int>(n), static_cast<int>(k),
                       static_cast<int>(E), kMoeBT, tok, pos, tiles, ntiles);
    if (int rc = check_hip(hipGetLastError(), "moe_sort launch")) return rc;
    const int64_t max_tiles = n / kMoeBT + std::min<int64_t>(E, n);

    GemmArgs a{};
    a.w = static_cast<const uint8_t*>(g.weight);
    a.s = static_cast<const uint8_t*>(g.scales);
    a.b = static_cast<const uint8_t*>(g.biases);
    a.w2 = static_cast<const uint8_t*>(u.weight);
    a.s2 = static_cast<const uint8_t*>(u.scales);
    a.b2 = static_cast<const uint8_t*>(u.biases);
    a.estride_w = g.weight_stride;
    a.estride_s = g.scale_stride;
    a.estride_b = g.bias_stride;
    a.x = static_cast<const uint16_t*>(x);
    a.y = hbuf;
    a.M = static_cast<int>(Fd);
    a.K = static_cast<int>(H);
    a.T = static_cast<int>(n);
    a.ldx = ldx;
    a.ldy = Fd;
    a.mtiles = static_cast<int>((Fd + 63) / 64);
    a.tiles = tiles;
    a.ntiles = ntiles;
    a.tok = tok;
    if (int rc = launch_sk<F, kMoeBT, kDualSilu>(a, static_cast<unsigned>(max_tiles * a.mtiles), stream)) return rc;

    GemmArgs b{};
    b.w = static_cast<const uint8_t*>(d.weight);
    b.s = static_cast<const uint8_t*>(d.scales);
    b.b = static_cast<const uint8_t*>(d.biases);
    b.w2 = b.w;
    b.s2 = b.s;
    b.b2 = b.b;
    b.estride_w = d.weight_stride;
    b.estride_s = d.scale_stride;
    b.estride_b = d.bias_stride;
    b.x = hbuf;  // h rows by position
    b.y = dbuf;
    b.M = static_cast<int>(H);
    b.K = static_cast<int>(Fd);
    b.T = static_cast<int>(n);
    b.ldx = Fd;
    b.ldy = H;
    b.mtiles = static_cast<int>((H + kBM - 1) / kBM);
    b.tiles = tiles;
    b.ntiles = ntiles;
    b.tok = nullptr;
    if (int rc = launch_sk<F, kMoeBT, kGather>(b, static_cast<unsigned>(max_tiles * b.mtiles), stream)) return rc;

    const int64_t threads = T * (H / 8);
    hipLaunchKernelGGL(moe_prefill_combine, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, stream,
                       dbuf, pos, static_cast<const uint16_t*>(rw), static_cast<int>(k), static_cast<int>(H),
                       static_cast<int>(T), static_cast<uint16_t*>(y), ldy);
    return check_hip(hipGetLastError(), "moe_prefill_combine launch");
}

}  // namespace
}  // namespace gdsllm

using namespace gdsllm;

namespace {

// Shared checks of the dense prefill entry points; returns 0 or an error code.
int check_dense(const std::string& n, const void* weight, const void* x, const void* y, int64_t out_dim, int64_t in_dim,
                int64_t tokens, int64_t ldx, int64_t ldy, bool& empty) {
    empty = false;
    if (out_dim < 0 || in_dim < 0 || tokens < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative dimension");
    if (in_dim % 32 != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": in_dim must be a multiple of 32, got " + std::to_string(in_dim));
    if (out_dim == 0 || in_dim == 0 || tokens == 0) {
        empty = true;
        return GDSLLM_OK;
    }
    if (!weight || !x || !y) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (ldx < in_dim || ldy < out_dim) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than the row length");
    if (out_dim > (int64_t(1) << 30) || in_dim > (int64_t(1) << 24) || tokens > (int64_t(1) << 24) || ldx > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": dimension too large");
    if (reinterpret_cast<uintptr_t>(weight) % 16 || reinterpret_cast<uintptr_t>(x) % 16 || ldx % 8 ||
        reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": weight and x rows must be 16-byte aligned (ldx % 8 == 0)");
    return GDSLLM_OK;
}

// The weight transfers address the rows of a tile (up to 256) by 32-bit
// offsets from the tile's first row: Q8_0 rows (in_dim * 34 / 32 bytes) must
// keep 255 rows + one stage within 4 GiB (in_dim below 15,852,288).
int check_q8_rows(const std::string& n, int64_t in_dim) {
    if (255 * (in_dim / 32 * 34) + 1024 >= (int64_t(1) << 32))
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": Q8_0 in_dim too large for the MFMA GEMM, got " +
                                                     std::to_string(in_dim));
    return GDSLLM_OK;
}

int off_grid(const std::string& n, int64_t in_dim) {
    return set_error(GDSLLM_ERR_UNSUPPORTED,
                     n + ": in_dim must be a multiple of 256 for the MFMA GEMM, got " + std::to_string(in_dim));
}

template <WF F>
int run_dense(const void* w, const void* s, const void* b, const void* x, void* y, int64_t M, int64_t K, int64_t T,
              int64_t ldx, int64_t ldy, void* stream) {
    GemmArgs a{};
    a.w = static_cast<const uint8_t*>(w);
    a.s = static_cast<const uint8_t*>(s);
    a.b = static_cast<const uint8_t*>(b);
    a.w2 = a.w;
    a.s2 = a.s;
    a.b2 = a.b;
    a.x = static_cast<const uint16_t*>(x);
    a.y = static_cast<uint16_t*>(y);
    a.M = static_cast<int>(M);
    a.K = static_cast<int>(K);
    a.T = static_cast<int>(T);
    a.ldx = ldx;
    a.ldy = ldy;
    const int rc = dense_gemm_auto<F>(a, as_stream(stream));
    return rc == GDSLLM_OK ? ok() : rc;
}

}  // namespace

extern "C" int gdsllm_dequant_gemm_q8_0(const void* weight, const void* x, void* y, int64_t out_dim, int64_t in_dim,
                                        int64_t tokens, int64_t ldx, int64_t ldy, void* stream) {
    bool empty;
    if (int rc = check_dense("dequant_gemm_q8_0", weight, x, y, out_dim, in_dim, tokens, ldx, ldy, empty)) return rc;
    if (empty) return ok();
    if (in_dim % 256 != 0) return off_grid("dequant_gemm_q8_0", in_dim);
    if (int rc = check_q8_rows("dequant_gemm_q8_0", in_dim)) return rc;
    return run_dense<WF::Q8_0>(weight, nullptr, nullptr, x, y, out_dim, in_dim, tokens, ldx, ldy, stream);
}

extern "C" int gdsllm_dequant_gemm_q4_0(const void* weight, const void* x, void* y, int64_t out_dim, int64_t in_dim,
                                        int64_t tokens, int64_t ldx, int64_t ldy, void* stream) {
    bool empty;
    if (int rc = check_dense("dequant_gemm_q4_0", weight, x, y, out_dim, in_dim, tokens, ldx, ldy, empty)) return rc;
    if (empty) return ok();
    if (in_dim % 256 == 0)
        return run_dense<WF::Q4_0>(weight, nullptr, nullptr, x, y, out_dim, in_dim, tokens, ldx, ldy, stream);
    // off the split-K grid: one Q4_0 block per K step
    const int r = dequant_gemm_q4_0_blockwise(weight, x, y, static_cast<int>(out_dim), static_cast<int>(in_dim),
                                              static_cast<int>(tokens), ldx, ldy, as_stream(stream));
    return r == GDSLLM_OK ? ok() : r;
}

extern "C" int gdsllm_dequant_gemm_affine_q4(const void* weight, const void* scales, const void* biases, const void* x,
                                             void* y, int64_t out_dim, int64_t in_dim, int64_t group_size,
                                             int64_t tokens, int64_t ldx, int64_t ldy, void* stream) {
    const std::string n = "dequant_gemm_affine_q4";
    if (group_size <= 0 || group_size % 8 != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": group_size must be a positive multiple of 8");
    bool empty;
    if (int rc = check_dense(n, weight, x, y, out_dim, in_dim, tokens, ldx, ldy, empty)) return rc;
    if (empty) return ok();
    if (in_dim % group_size != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": in_dim must be a multiple of group_size");
    if (in_dim % 256 != 0) return off_grid(n, in_dim);
    if (!scales || !biases) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (group_size != 32 && group_size != 64 && group_size != 128)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": the MFMA GEMM takes group_size 32, 64 or 128");
    const uintptr_t sal = group_size == 32 ? 16 : 4;
    if (reinterpret_cast<uintptr_t>(scales) % sal || reinterpret_cast<uintptr_t>(biases) % sal)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": scales/biases must be " + std::to_string(sal) + "-byte aligned");
    switch (group_size) {
        case 32: return run_dense<WF::AFF32>(weight, scales, biases, x, y, out_dim, in_dim, tokens, ldx, ldy, stream);
        case 64: return run_dense<WF::AFF64>(weight, scales, biases, x, y, out_dim, in_dim, tokens, ldx, ldy, stream);
        default: return run_dense<WF::AFF128>(weight, scales, biases, x, y, out_dim, in_dim, tokens, ldx, ldy, stream);
    }
}

extern "C" size_t gdsllm_moe_prefill_workspace_size(int64_t tokens, int64_t top_k, int64_t ffn_dim, int64_t hidden,
                                                    int64_t num_experts) {
    if (tokens < 0 || top_k < 0 || ffn_dim < 0 || hidden < 0 || num_experts < 0) return 0;
    return prefill_layout(tokens, top_k, ffn_dim, hidden, num_experts).total;
}

extern "C" int gdsllm_moe_prefill_affine_q4(const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                                            const gdsllm_affine_experts* down, const void* x, int64_t ldx,
                                            const int32_t* idx, const void* routing_weights, int64_t tokens,
                                            int64_t top_k, void* y, int64_t ldy, void* workspace,
                                            size_t workspace_bytes, void* stream) {
    const std::string n = "moe_prefill_affine_q4";
    const gdsllm_affine_experts* ps[3] = {gate, up, down};
    const char* names[3] = {"gate", "up", "down"};
    for (int i = 0; i < 3; ++i) {
        const gdsllm_affine_experts* p = ps[i];
        if (!p) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": " + names[i] + " is null");
        if (!p->weight || !p->scales || !p->biases) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": " + names[i] + ": null pointer");
        if (p->num_experts <= 0 || p->out_dim <= 0 || p->in_dim <= 0 || p->group_size <= 0)
            return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": " + names[i] + ": non-positive size");
        if (p->in_dim % p->group_size != 0 || p->group_size % 8 != 0)
            return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": " + names[i] + ": in_dim must be a multiple of group_size");
    }
    const int64_t E = gate->num_experts, H = gate->in_dim, Fd = gate->out_dim, g = gate->group_size;
    if (up->in_dim != H || up->out_dim != Fd || down->in_dim != Fd || down->out_dim != H || up->group_size != g ||
        down->group_size != g || up->num_experts != E || down->num_experts != E)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": gate/up [E,F,H] and down [E,H,F] shapes disagree");
    if (gate->weight_stride != up->weight_stride || gate->scale_stride != up->scale_stride ||
        gate->bias_stride != up->bias_stride)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": gate and up pools must have the same expert strides");
    if (tokens < 0 || top_k < 1 || top_k > 64)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": tokens must be >= 0 and top_k in [1, 64]");
    if (tokens == 0) return ok();
    if (!x || !idx || !routing_weights || !y || !workspace) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (ldx < H || ldy < H) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": ldx/ldy smaller than hidden");
    if (workspace_bytes < gdsllm_moe_prefill_workspace_size(tokens, top_k, Fd, H, E))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": workspace too small");
    if (E > kSortMaxExperts || tokens * top_k > (int64_t(1) << 24) || H > (int64_t(1) << 20) || Fd > (int64_t(1) << 20))
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": at most 4096 experts, 2^24 routed entries, dimensions <= 2^20");
    // X rows are addressed with 32-bit byte offsets: token * ldx and position * ffn
    if (tokens * ldx * 2 >= (int64_t(1) << 32) || tokens * top_k * Fd * 2 >= (int64_t(1) << 32))
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": activations beyond 4 GiB");
    if (H % 256 != 0 || Fd % 256 != 0 || (g != 32 && g != 64 && g != 128))
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": hidden and ffn must be multiples of 256, group_size 32, 64 or 128");
    const uintptr_t sal = g == 32 ? 16 : 4;
    for (const gdsllm_affine_experts* p : ps)
        if (reinterpret_cast<uintptr_t>(p->weight) % 16 || p->weight_stride % 16 ||
            reinterpret_cast<uintptr_t>(p->scales) % sal || reinterpret_cast<uintptr_t>(p->biases) % sal ||
            p->scale_stride % static_cast<int64_t>(sal) || p->bias_stride % static_cast<int64_t>(sal))
            return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": expert words must be 16-byte aligned, scales/biases " +
                                                         std::to_string(sal) + "-byte");
    if (reinterpret_cast<uintptr_t>(x) % 16 || ldx % 8 || reinterpret_cast<uintptr_t>(y) % 16 || ldy % 8 ||
        reinterpret_cast<uintptr_t>(routing_weights) % 2 || reinterpret_cast<uintptr_t>(idx) % 4 ||
        reinterpret_cast<uintptr_t>(workspace) % 256)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": x and y rows must be 16-byte aligned, workspace 256-byte");
    const hipStream_t s = as_stream(stream);
    auto* ws = static_cast<uint8_t*>(workspace);
    int rc;
    switch (g) {
        case 32: rc = moe_prefill_run<WF::AFF32>(*gate, *up, *down, x, ldx, idx, routing_weights, tokens, top_k, y, ldy, ws, s); break;
        case 64: rc = moe_prefill_run<WF::AFF64>(*gate, *up, *down, x, ldx, idx, routing_weights, tokens, top_k, y, ldy, ws, s); break;
        default: rc = moe_prefill_run<WF::AFF128>(*gate, *up, *down, x, ldx, idx, routing_weights, tokens, top_k, y, ldy, ws, s); break;
    }
    return rc == GDSLLM_OK ? ok() : rc;
}

namespace {
template <WF F>
int gate_up_silu_entry(const std::string& n, const void* gate, const void* up, const void* x, void* h,
                       int64_t ffn_dim, int64_t in_dim, int64_t tokens, int64_t ldx, int64_t ldh, void* stream) {
    bool empty;
    if (int rc = check_dense(n, gate, x, h, ffn_dim, in_dim, tokens, ldx, ldh, empty)) return rc;
    if (empty) return ok();
    if (!up) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (reinterpret_cast<uintptr_t>(up) % 16)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": weight and x rows must be 16-byte aligned (ldx % 8 == 0)");
    if (in_dim % 256 != 0) return off_grid(n, in_dim);
    if (F == WF::Q8_0)
        if (int rc = check_q8_rows(n, in_dim)) return rc;
    GemmArgs a{};
    a.w = static_cast<const uint8_t*>(gate);
    a.w2 = static_cast<const uint8_t*>(up);
    a.x = static_cast<const uint16_t*>(x);
    a.y = static_cast<uint16_t*>(h);
    a.M = static_cast<int>(ffn_dim);
    a.K = static_cast<int>(in_dim);
    a.T = static_cast<int>(tokens);
    a.ldx = ldx;
    a.ldy = ldh;
    const int rc = dense_dual_gemm_auto<F>(a, as_stream(stream));
    return rc == GDSLLM_OK ? ok() : rc;
}
}  // namespace

extern "C" int gdsllm_dequant_gemm_gate_up_silu_q4_0(const void* gate_weight, const void* up_weight, const void* x,
                                                     void* h, int64_t ffn_dim, int64_t in_dim, int64_t tokens,
                                                     int64_t ldx, int64_t ldh, void* stream) {
    return gate_up_silu_entry<WF::Q4_0>("dequant_gemm_gate_up_silu_q4_0", gate_weight, up_weight, x, h, ffn_dim,
                                        in_dim, tokens, ldx, ldh, stream);
}

extern "C" int gdsllm_dequant_gemm_gate_up_silu_q8_0(const void* gate_weight, const void* up_weight, const void* x,
                                                     void* h, int64_t ffn_dim, int64_t in_dim, int64_t tokens,
                                                     int64_t ldx, int64_t ldh, void* stream) {
    return gate_up_silu_entry<WF::Q8_0>("dequant_gemm_gate_up_silu_q8_0", gate_weight, up_weight, x, h, ffn_dim,
                                        in_dim, tokens, ldx, ldh, stream);
}
