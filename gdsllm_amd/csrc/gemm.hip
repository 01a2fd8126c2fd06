// Prefill dequant-GEMM for GGUF Q4_0 weights on the gfx950 matrix cores.
//
// Y[t][r] = fp16( sum_k X[t][k] * W[r][k] ) for a chunk of T prompt tokens:
// what the reference's prefill branch computes as dequant -> F.linear
// (runtime/llama.py:160-166), fused so the fp16 weight matrix never goes back
// to HBM.  W enters the matrix cores as the bit-exact fp16 dequantized value
// d*(q-8) (the same fp16 tensor the reference hands to cuBLAS), X as fp16,
// accumulation in fp32 (v_mfma_f32_16x16x32_f16), one fp16 rounding at the end.
//
// Tiling: a workgroup owns a BT x BM output tile and walks K in steps of 64
// (two Q4_0 blocks = 36 bytes per weight row, 4-byte aligned when
// in_dim % 64 == 0).  Each step stages the fp16 X tile and the dequantized W
// tile in LDS (rows padded to 144 B = 4*9 dwords: conflict-free ds_read_b128),
// while the next step's global data is already in flight in registers.
// A wave computes a (BT/WT) x (BM/WM) sub-tile from 16x16 MFMA fragments.
//
// MFMA operand layout (16x16x32 f16): lane l holds A row (l % 16) and B column
// (l % 16), eight consecutive k values 8*(l/16)..+7 of each; the result holds
// D[4*(l/16) + v][l % 16] in its four fp32 registers.

#include "common.h"

namespace gdsllm {
namespace {

constexpr int BK = 64;             // k per pipeline step (2 Q4_0 blocks)
constexpr int kPadHalves = BK + 8; // LDS row stride in fp16 (144 B)

template <int BT, int BM, int WT, int WM>
struct Tile {
    static constexpr int kThreads = WT * WM * 64;
    static constexpr int kWaveT = BT / WT;  // tokens per wave
    static constexpr int kWaveM = BM / WM;  // weight rows per wave
    static constexpr int kFragT = kWaveT / 16;
    static constexpr int kFragM = kWaveM / 16;
    static constexpr int kXChunks = BT * BK / 8 / kThreads;  // 16-byte X chunks per thread per step
    static_assert(BT * BK / 8 % kThreads == 0, "X tile must split evenly");
    static_assert(BM * 2 == kThreads, "two threads dequantize one weight row (one block each)");
};

// fp16 pair (lo, hi) -> bit-exact dequantized pair d*(q-8) given the biased
// nibble pair `p` (1024+q or 64+q per half) and the bias `off` to remove.
__device__ __forceinline__ uint32_t dq_pair(uint32_t p, half2_t off, half2_t dd) {
    const half2_t q = __builtin_bit_cast(half2_t, p) + off;  // exact: q - 8
    return __builtin_bit_cast(uint32_t, q * dd);             // one RNE rounding
}

template <int BT, int BM, int WT, int WM>
__global__ __launch_bounds__(WT * WM * 64) void dequant_gemm_q4_0(const uint8_t* __restrict__ W,
                                                                  const uint16_t* __restrict__ X,
                                                                  uint16_t* __restrict__ Y, int M, int K, int T,
                                                                  int64_t ldx, int64_t ldy) {
    using TL = Tile<BT, BM, WT, WM>;
    __shared__ __attribute__((aligned(16))) uint16_t Xs[BT * kPadHalves];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[BM * kPadHalves];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wt = wave / WM, wm = wave % WM;
    const int t0 = blockIdx.y * BT;
    const int m0 = blockIdx.x * BM;
    const int64_t row_bytes = static_cast<int64_t>(K / 32) * 18;
    const int nsteps = (K + BK - 1) / BK;

    // this thread's weight row and block within the step
    const int wr = tid >> 1, wh = tid & 1;
    const bool w_live = (m0 + wr) < M;
    const uint32_t* wrow = reinterpret_cast<const uint32_t*>(W + static_cast<int64_t>(m0 + (w_live ? wr : 0)) * row_bytes);

    uint4 xpre[TL::kXChunks];
    uint32_t wpre[9];

    auto load_step = [&](int s) {
        const int k0 = s * BK;
#pragma unroll
        for (int i = 0; i < TL::kXChunks; ++i) {
            const int c = tid + i * TL::kThreads;
            const int row = c / (BK / 8), piece = c % (BK / 8);
            const int t = t0 + row, k = k0 + 8 * piece;
            xpre[i] = (t < T && k < K) ? *reinterpret_cast<const uint4*>(X + t * ldx + k) : make_uint4(0, 0, 0, 0);
        }
        // two blocks = 36 bytes = 9 dwords (rows of a K % 64 == 0 matrix are 36n bytes)
#pragma unroll
        for (int i = 0; i < 9; ++i) wpre[i] = w_live ? __builtin_nontemporal_load(wrow + s * 9 + i) : 0u;
    };

    auto store_step = [&]() {
#pragma unroll
        for (int i = 0; i < TL::kXChunks; ++i) {
            const int c = tid + i * TL::kThreads;
            const int row = c / (BK / 8), piece = c % (BK / 8);
            *reinterpret_cast<uint4*>(&Xs[row * kPadHalves + 8 * piece]) = xpre[i];
        }
        // dequantize block wh of this thread's row: elements j (low nibble of
        // qs[j]) and j+16 (high nibble), j = 0..15, in natural k order
        uint32_t dbits, q[4];
        if (wh == 0) {
            dbits = wpre[0] & 0xFFFFu;
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = align2(wpre[i], wpre[i + 1]);
        } else {
            dbits = wpre[4] >> 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = wpre[5 + i];
        }
        const half_t dh = __builtin_bit_cast(half_t, static_cast<uint16_t>(dbits));
        const half2_t dd = {dh, dh};
        const half2_t off_lo = {static_cast<half_t>(-1032.0f), static_cast<half_t>(-1032.0f)};
        const half2_t off_hi = {static_cast<half_t>(-72.0f), static_cast<half_t>(-72.0f)};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // spread bytes (b0, b1) and (b2, b3) into the low byte of each half
            const uint32_t t01 = __builtin_amdgcn_perm(0u, q[i], 0x0C010C00u);
            const uint32_t t23 = __builtin_amdgcn_perm(0u, q[i], 0x0C030C02u);
            lo[2 * i] = dq_pair(nib_lo_pair(t01), off_lo, dd);
            lo[2 * i + 1] = dq_pair(nib_lo_pair(t23), off_lo, dd);
            hi[2 * i] = dq_pair(nib_hi_pair(t01), off_hi, dd);
            hi[2 * i + 1] = dq_pair(nib_hi_pair(t23), off_hi, dd);
        }
        uint16_t* dst = &Ws[wr * kPadHalves + 32 * wh];
        *reinterpret_cast<uint4*>(dst) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<uint4*>(dst + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        *reinterpret_cast<uint4*>(dst + 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *reinterpret_cast<uint4*>(dst + 24) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    };

    float4_t acc[TL::kFragT][TL::kFragM];
#pragma unroll
    for (int a = 0; a < TL::kFragT; ++a)
#pragma unroll
        for (int b = 0; b < TL::kFragM; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int fi = lane & 15, fg = lane >> 4;
    load_step(0);
    for (int s = 0; s < nsteps; ++s) {
        __syncthreads();
        store_step();
        __syncthreads();
        if (s + 1 < nsteps) load_step(s + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            half8_t af[TL::kFragT], bf[TL::kFragM];
#pragma unroll
            for (int a = 0; a < TL::kFragT; ++a)
                af[a] = *reinterpret_cast<const half8_t*>(&Xs[(wt * TL::kWaveT + 16 * a + fi) * kPadHalves + 32 * kk + 8 * fg]);
#pragma unroll
            for (int b = 0; b < TL::kFragM; ++b)
                bf[b] = *reinterpret_cast<const half8_t*>(&Ws[(wm * TL::kWaveM + 16 * b + fi) * kPadHalves + 32 * kk + 8 * fg]);
#pragma unroll
            for (int a = 0; a < TL::kFragT; ++a)
#pragma unroll
                for (int b = 0; b < TL::kFragM; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
    }

#pragma unroll
    for (int a = 0; a < TL::kFragT; ++a)
#pragma unroll
        for (int b = 0; b < TL::kFragM; ++b) {
            const int m = m0 + wm * TL::kWaveM + 16 * b + fi;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int t = t0 + wt * TL::kWaveT + 16 * a + 4 * fg + v;
                if (t < T && m < M) Y[t * ldy + m] = f2h_bits(acc[a][b][v]);
            }
        }
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
    // A K % 64 == 32 row is 18*(2n+1) bytes, so rows after the first start off
    // the dword grid the two-block loads use.
    if (in_dim % 64 != 0) return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": in_dim must be a multiple of 64");
    if (reinterpret_cast<uintptr_t>(weight) % 4 || reinterpret_cast<uintptr_t>(x) % 16 || ldx % 8 ||
        reinterpret_cast<uintptr_t>(y) % 2)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": weight must be 4-byte aligned and x rows 16-byte aligned");
    constexpr int BT = 64, BM = 128, WT = 2, WM = 2;
    dim3 grid(static_cast<unsigned>((out_dim + BM - 1) / BM), static_cast<unsigned>((tokens + BT - 1) / BT));
    hipLaunchKernelGGL((dequant_gemm_q4_0<BT, BM, WT, WM>), grid, dim3(WT * WM * 64), 0, as_stream(stream),
                       static_cast<const uint8_t*>(weight), static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y),
                       static_cast<int>(out_dim), static_cast<int>(in_dim), static_cast<int>(tokens), ldx, ldy);
    if (int rc = check_hip(hipGetLastError(), "dequant_gemm_q4_0 launch")) return rc;
    return ok();
}
