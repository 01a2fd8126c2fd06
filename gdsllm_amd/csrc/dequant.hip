// Bit-exact fp16 dequantization of GGUF Q4_0 / Q8_0 blocks and affine-Q4
// groups (the reference's runtime/gguf_dequant.cu and the dequant half of
// runtime/affine_q4_dequant.cu).
//
// Each output element is ONE round-to-nearest-even to fp16 of the fp32 value
// the reference forms: d*(q-8) and d*q are exact in fp32 (11-bit by 5/8-bit
// products), nib*s+b is an exact product plus one fp32 rounding.  HBM-bound:
// 18 (or 34) bytes in and 64 bytes out per 32 weights.  The GGUF kernels give
// every lane one 16-byte output chunk (8 weights) at a time, so each store
// instruction of a wave writes 1 KiB of contiguous output, and the lane reads
// the 2 + 8 source bytes its chunk needs with dword loads that neighbouring
// lanes share through the cache.
#include "common.h"

namespace gdsllm {
namespace {

constexpr int kThreads = 256;

// ---- Q4_0 -------------------------------------------------------------------
// Block: fp16 d, then 16 bytes qs; element j = d*((qs[j] & 15) - 8),
// element j+16 = d*((qs[j] >> 4) - 8)  (runtime/gguf_dequant.cu:84-107).
__device__ __forceinline__ void q4_block_to_fp16(uint32_t d_bits, const uint32_t q[4], uint32_t out[16]) {
    const float d = h2f(d_bits);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t lo2[2], hi2[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t b0 = (q[w] >> (16 * p)) & 0xFFu;
            const uint32_t b1 = (q[w] >> (16 * p + 8)) & 0xFFu;
            const uint16_t l0 = f2h_bits(fp32_rounded(d * static_cast<float>(static_cast<int>(b0 & 15u) - 8)));
            const uint16_t l1 = f2h_bits(fp32_rounded(d * static_cast<float>(static_cast<int>(b1 & 15u) - 8)));
            const uint16_t h0 = f2h_bits(fp32_rounded(d * static_cast<float>(static_cast<int>(b0 >> 4) - 8)));
            const uint16_t h1 = f2h_bits(fp32_rounded(d * static_cast<float>(static_cast<int>(b1 >> 4) - 8)));
            lo2[p] = static_cast<uint32_t>(l0) | (static_cast<uint32_t>(l1) << 16);
            hi2[p] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
        }
        out[2 * w] = lo2[0];
        out[2 * w + 1] = lo2[1];
        out[8 + 2 * w] = hi2[0];
        out[8 + 2 * w + 1] = hi2[1];
    }
}

// One block per thread, byte loads: any alignment, any count (tail / odd cases).
__global__ __launch_bounds__(kThreads) void dequant_q4_0_bytes(const uint8_t* __restrict__ src,
                                                                uint16_t* __restrict__ dst,
                                                                int64_t first, int64_t num_blocks) {
    const int64_t b = first + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (b >= num_blocks) return;
    const uint8_t* s = src + b * 18;
    const float d = h2f(static_cast<uint32_t>(s[0]) | (static_cast<uint32_t>(s[1]) << 8));
    uint16_t* o = dst + b * 32;
    for (int j = 0; j < 16; ++j) {
        const int byte = s[2 + j];
        o[j] = f2h_bits(fp32_rounded(d * static_cast<float>((byte & 15) - 8)));
        o[j + 16] = f2h_bits(fp32_rounded(d * static_cast<float>((byte >> 4) - 8)));
    }
}

// ---- Q8_0 -------------------------------------------------------------------
// Block: fp16 d, then int8 qs[32]; element i = d*qs[i] (runtime/gguf_dequant.cu:40-57).
__device__ __forceinline__ void q8_block_to_fp16(uint32_t d_bits, const uint32_t q[8], uint4* out) {
    const float d = h2f(d_bits);
#pragma unroll
    for (int w = 0; w < 8; w += 2) {
        uint32_t o[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t v = q[w + h];
            const float a = fp32_rounded(d * static_cast<float>(static_cast<int8_t>(v & 0xFFu)));
            const float b = fp32_rounded(d * static_cast<float>(static_cast<int8_t>((v >> 8) & 0xFFu)));
            const float c = fp32_rounded(d * static_cast<float>(static_cast<int8_t>((v >> 16) & 0xFFu)));
            const float e = fp32_rounded(d * static_cast<float>(static_cast<int8_t>(v >> 24)));
            o[2 * h] = static_cast<uint32_t>(f2h_bits(a)) | (static_cast<uint32_t>(f2h_bits(b)) << 16);
            o[2 * h + 1] = static_cast<uint32_t>(f2h_bits(c)) | (static_cast<uint32_t>(f2h_bits(e)) << 16);
        }
        out[w / 2] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

__global__ __launch_bounds__(kThreads) void dequant_q8_0_bytes(const uint8_t* __restrict__ src,
                                                                uint16_t* __restrict__ dst,
                                                                int64_t first, int64_t num_blocks) {
    const int64_t b = first + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (b >= num_blocks) return;
    const uint8_t* s = src + b * 34;
    const float d = h2f(static_cast<uint32_t>(s[0]) | (static_cast<uint32_t>(s[1]) << 8));
    uint16_t* o = dst + b * 32;
    for (int j = 0; j < 32; ++j) o[j] = f2h_bits(fp32_rounded(d * static_cast<float>(static_cast<int8_t>(s[2 + j]))));
}

// ---- GGUF, one 16-byte output chunk per lane ------------------------------------
// Chunk u holds output elements [8u, 8u + 8): part p = u % 4 of block u / 4.
// Q4_0: parts 0 / 1 are the low nibbles of code bytes 0-7 / 8-15, parts 2 / 3
// their high nibbles (element j <- qs[j] & 15, element j + 16 <- qs[j] >> 4,
// runtime/gguf_dequant.cu:105-106).  Q8_0: part p is code bytes 8p .. 8p + 7.
//
// Arithmetic, exact up to the one rounding the reference performs: a code
// pair becomes two fp16 values with one v_perm and one mask, 1024 + q (low
// nibble or biased byte) or 64 + q (high nibble); one packed subtract of
// 1032 / 72 / 1152 gives q - 8 or q exactly; one packed multiply by d rounds
// the exact product d*(q - 8) (d*q) once to fp16 -- the reference's
// __float2half of the exact fp32 product, signed zeros, subnormals, overflow
// to inf and NaN included.
constexpr int kChunksPerThread = 4;  // chunks u, u + 256, u + 512, u + 768 of the workgroup's 1024

// Blocks start 2 bytes off a dword boundary when their index is odd (18 and
// 34 are 2 mod 4), so d sits in the high half of the dword below it, and the
// codes start on a dword boundary; for even blocks it is the other way round.
template <bool Q8>
__device__ __forceinline__ void gguf_chunk_load(const uint8_t* __restrict__ src, int64_t u, uint32_t& d_bits,
                                                uint32_t& c0, uint32_t& c1) {
    constexpr int kBlockBytes = Q8 ? 34 : 18;
    const int64_t b = u >> 2;
    const int p = static_cast<int>(u & 3);
    const int64_t o = b * kBlockBytes;
    const uint32_t dw = *reinterpret_cast<const uint32_t*>(src + (o & ~int64_t(3)));
    d_bits = (dw >> (8 * (o & 2))) & 0xFFFFu;
    // codes: bytes [s, s + 8), s = 0 or 2 mod 4.  Two dwords from s rounded
    // down, and the last two code bytes by a 16-bit load (so nothing past the
    // block is read); v_alignbyte by 0 or 2 picks the 8 bytes, no branch.
    const int64_t s = o + 2 + 8 * (Q8 ? p : (p & 1));
    const uint32_t sh = static_cast<uint32_t>(s & 2);
    const uint32_t* a = reinterpret_cast<const uint32_t*>(src + (s & ~int64_t(3)));
    const uint32_t x0 = a[0], x1 = a[1];
    const uint32_t t = *reinterpret_cast<const uint16_t*>(src + s + 6);
    c0 = __builtin_amdgcn_alignbyte(x1, x0, sh);
    c1 = __builtin_amdgcn_alignbyte(t, x1, sh);
}

// Code bytes j, j + 1 of `c` as fp16 pair halves {0x64 | byte} or, for high
// nibbles, {0x54 | byte}, masked to the field (bytes 0-1: sel kSelB01, 2-3: kSelB23).
constexpr uint32_t kSelB01 = 0x04010400u, kSelB23 = 0x04030402u;

template <bool Q8>
__device__ __forceinline__ uint4 gguf_chunk_values(uint32_t d_bits, uint32_t c0, uint32_t c1, int part) {
    const half_t dh = __builtin_bit_cast(half_t, static_cast<uint16_t>(d_bits));
    const half2_t d2 = {dh, dh};
    uint32_t pr[4];
    if constexpr (Q8) {
        const uint32_t u0 = c0 ^ 0x80808080u, u1 = c1 ^ 0x80808080u;
        pr[0] = __builtin_amdgcn_perm(0x64646464u, u0, kSelB01);
        pr[1] = __builtin_amdgcn_perm(0x64646464u, u0, kSelB23);
        pr[2] = __builtin_amdgcn_perm(0x64646464u, u1, kSelB01);
        pr[3] = __builtin_amdgcn_perm(0x64646464u, u1, kSelB23);
    } else {
        const bool high = part >= 2;
        const uint32_t ex = high ? 0x54545454u : 0x64646464u;
        const uint32_t mask = high ? 0x54F054F0u : 0x640F640Fu;
        pr[0] = __builtin_amdgcn_perm(ex, c0, kSelB01) & mask;
        pr[1] = __builtin_amdgcn_perm(ex, c0, kSelB23) & mask;
        pr[2] = __builtin_amdgcn_perm(ex, c1, kSelB01) & mask;
        pr[3] = __builtin_amdgcn_perm(ex, c1, kSelB23) & mask;
    }
    const half_t bias = Q8 ? static_cast<half_t>(1152.0f) : (part >= 2 ? static_cast<half_t>(72.0f)
                                                                        : static_cast<half_t>(1032.0f));
    const half2_t b2 = {bias, bias};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        half2_t q = __builtin_bit_cast(half2_t, pr[i]) - b2;  // exact: q - 8 (Q4_0) or q (Q8_0)
        o[i] = __builtin_bit_cast(uint32_t, q * d2);         // one rounding of the exact product
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// `src` 4-byte aligned, `dst` 16-byte aligned; num_chunks = 4 * blocks.
template <bool Q8>
__global__ __launch_bounds__(kThreads) void dequant_gguf_chunks(const uint8_t* __restrict__ src,
                                                                 uint4* __restrict__ dst, int64_t num_chunks) {
    const int64_t u0 = static_cast<int64_t>(blockIdx.x) * (kThreads * kChunksPerThread) + threadIdx.x;
    uint32_t d[kChunksPerThread], c0[kChunksPerThread], c1[kChunksPerThread];
    if (static_cast<int64_t>(blockIdx.x + 1) * (kThreads * kChunksPerThread) <= num_chunks) {
        // every chunk of the workgroup exists: all loads in flight, then all stores
#pragma unroll
        for (int i = 0; i < kChunksPerThread; ++i) gguf_chunk_load<Q8>(src, u0 + i * kThreads, d[i], c0[i], c1[i]);
#pragma unroll
        for (int i = 0; i < kChunksPerThread; ++i)
            dst[u0 + i * kThreads] = gguf_chunk_values<Q8>(d[i], c0[i], c1[i], static_cast<int>((u0 + i * kThreads) & 3));
        return;
    }
#pragma unroll
    for (int i = 0; i < kChunksPerThread; ++i) {
        const int64_t u = u0 + i * kThreads;
        if (u < num_chunks) {
            gguf_chunk_load<Q8>(src, u, d[i], c0[i], c1[i]);
            dst[u] = gguf_chunk_values<Q8>(d[i], c0[i], c1[i], static_cast<int>(u & 3));
        }
    }
}

// ---- token-row gather (embedding lookup) ----------------------------------------
// Row ids[t] of a [vocab][hidden] GGUF table, dequantized into out[t][hidden]
// with the same per-element rounding as above: F.embedding over the dequantized
// table (runtime/scheduler.py:22-35) without dequantizing the other rows.
// grid.y = token, grid.x covers the row's block pairs (hidden % 64 == 0, the
// table 4-byte aligned); ids outside [0, vocab) give a zero row.
template <bool Q8>
__global__ __launch_bounds__(kThreads) void embed_rows_pairs(const uint8_t* __restrict__ table,
                                                              const int64_t* __restrict__ ids, int64_t vocab,
                                                              int64_t hidden, uint4* __restrict__ out) {
    const int64_t t = blockIdx.y;
    const int64_t pairs = hidden / 64;
    const int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (p >= pairs) return;
    const int64_t id = ids[t];
    uint4* o = out + (t * hidden + 64 * p) / 8;
    if (id < 0 || id >= vocab) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = make_uint4(0, 0, 0, 0);
        return;
    }
    constexpr int kPairDw = Q8 ? 17 : 9;
    const uint32_t* s =
        reinterpret_cast<const uint32_t*>(table + id * (hidden / 32) * (Q8 ? 34 : 18)) + p * kPairDw;
    uint32_t v[kPairDw];
#pragma unroll
    for (int i = 0; i < kPairDw; ++i) v[i] = s[i];
    if constexpr (Q8) {
        uint32_t q0[8], q1[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            q0[i] = align2(v[i], v[i + 1]);
            q1[i] = v[9 + i];
        }
        q8_block_to_fp16(v[0] & 0xFFFFu, q0, o);
        q8_block_to_fp16(v[8] >> 16, q1, o + 4);
    } else {
        uint32_t q0[4] = {align2(v[0], v[1]), align2(v[1], v[2]), align2(v[2], v[3]), align2(v[3], v[4])};
        uint32_t q1[4] = {v[5], v[6], v[7], v[8]};
        uint32_t w[16];
        q4_block_to_fp16(v[0] & 0xFFFFu, q0, w);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
        q4_block_to_fp16(v[4] >> 16, q1, w);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[4 + i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    }
}

// ---- affine Q4 --------------------------------------------------------------
// Word w holds elements 8w..8w+7, nibble n = (word >> 4n) & 15 (LSB first);
// group = element / group_size over the flat index; value = nib*s + b in fp32,
// then one fp16 rounding (runtime/affine_q4_dequant.cu:28-59).  A thread takes
// words i, i + 256, i + 512, i + 768 of its workgroup's 1024: coalesced dword
// loads and 16-byte stores.  The group of a word is a shift when
// words_per_group is a power of two (every converter group size), else a
// division.
template <bool POW2>
__global__ __launch_bounds__(kThreads) void dequant_affine_words(const uint32_t* __restrict__ w,
                                                                  const uint16_t* __restrict__ scales,
                                                                  const uint16_t* __restrict__ biases,
                                                                  uint4* __restrict__ dst,
                                                                  int64_t num_words, int words_per_group,
                                                                  int group_shift) {
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * (kThreads * kChunksPerThread) + threadIdx.x;
    uint32_t v[kChunksPerThread], sb[kChunksPerThread][2];
#pragma unroll
    for (int k = 0; k < kChunksPerThread; ++k) {
        const int64_t i = i0 + k * kThreads;
        if (i < num_words) {
            const int64_t g = POW2 ? (i >> group_shift) : i / words_per_group;
            v[k] = __builtin_nontemporal_load(w + i);
            sb[k][0] = scales[g];
            sb[k][1] = biases[g];
        }
    }
#pragma unroll
    for (int k = 0; k < kChunksPerThread; ++k) {
        const int64_t i = i0 + k * kThreads;
        if (i < num_words) {
            const float sc = h2f(sb[k][0]), bi = h2f(sb[k][1]);
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = fp32_rounded(static_cast<float>((v[k] >> (8 * j)) & 15u) * sc + bi);
                const float hi = fp32_rounded(static_cast<float>((v[k] >> (8 * j + 4)) & 15u) * sc + bi);
                o[j] = static_cast<uint32_t>(f2h_bits(lo)) | (static_cast<uint32_t>(f2h_bits(hi)) << 16);
            }
            dst[i] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// Destination not 16-byte aligned: one thread per element.
__global__ __launch_bounds__(kThreads) void dequant_affine_elems(const uint32_t* __restrict__ w,
                                                                  const uint16_t* __restrict__ scales,
                                                                  const uint16_t* __restrict__ biases,
                                                                  uint16_t* __restrict__ dst,
                                                                  int64_t num_elements, int group_size) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= num_elements) return;
    const int64_t g = i / group_size;
    const uint32_t nib = (w[i >> 3] >> (4 * (i & 7))) & 15u;
    dst[i] = f2h_bits(fp32_rounded(static_cast<float>(nib) * h2f(scales[g]) + h2f(biases[g])));
}

int grid_for(int64_t n) { return static_cast<int>((n + kThreads - 1) / kThreads); }

}  // namespace
}  // namespace gdsllm

using namespace gdsllm;

extern "C" int gdsllm_dequant_q4_0(const void* src, void* dst, int64_t num_blocks, void* stream) {
    if (num_blocks < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_q4_0: negative block count");
    if (num_blocks == 0) return ok();
    if (!src || !dst) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_q4_0: null pointer");
    if (num_blocks > (int64_t(1) << 36)) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_q4_0: block count too large");
    hipStream_t s = as_stream(stream);
    const bool aligned = (reinterpret_cast<uintptr_t>(src) % 4 == 0) && (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
    int64_t done = 0;
    if (aligned) {
        const int64_t chunks = 4 * num_blocks;
        const int64_t per_wg = kThreads * kChunksPerThread;
        hipLaunchKernelGGL(dequant_gguf_chunks<false>, dim3(static_cast<unsigned>((chunks + per_wg - 1) / per_wg)),
                           dim3(kThreads), 0, s, static_cast<const uint8_t*>(src), static_cast<uint4*>(dst), chunks);
        done = num_blocks;
    }
    if (done < num_blocks) {
        hipLaunchKernelGGL(dequant_q4_0_bytes, dim3(grid_for(num_blocks - done)), dim3(kThreads), 0, s,
                           static_cast<const uint8_t*>(src), static_cast<uint16_t*>(dst), done, num_blocks);
    }
    if (int rc = check_hip(hipGetLastError(), "dequant_q4_0 launch")) return rc;
    return ok();
}

extern "C" int gdsllm_dequant_q8_0(const void* src, void* dst, int64_t num_blocks, void* stream) {
    if (num_blocks < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_q8_0: negative block count");
    if (num_blocks == 0) return ok();
    if (!src || !dst) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_q8_0: null pointer");
    if (num_blocks > (int64_t(1) << 36)) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_q8_0: block count too large");
    hipStream_t s = as_stream(stream);
    const bool aligned = (reinterpret_cast<uintptr_t>(src) % 4 == 0) && (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
    int64_t done = 0;
    if (aligned) {
        const int64_t chunks = 4 * num_blocks;
        const int64_t per_wg = kThreads * kChunksPerThread;
        hipLaunchKernelGGL(dequant_gguf_chunks<true>, dim3(static_cast<unsigned>((chunks + per_wg - 1) / per_wg)),
                           dim3(kThreads), 0, s, static_cast<const uint8_t*>(src), static_cast<uint4*>(dst), chunks);
        done = num_blocks;
    }
    if (done < num_blocks) {
        hipLaunchKernelGGL(dequant_q8_0_bytes, dim3(grid_for(num_blocks - done)), dim3(kThreads), 0, s,
                           static_cast<const uint8_t*>(src), static_cast<uint16_t*>(dst), done, num_blocks);
    }
    if (int rc = check_hip(hipGetLastError(), "dequant_q8_0 launch")) return rc;
    return ok();
}

extern "C" int gdsllm_dequant_affine_q4(const void* weight, const void* scales, const void* biases,
                                        void* dst, int64_t num_elements, int64_t in_dim,
                                        int64_t group_size, void* stream) {
    if (num_elements < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_affine_q4: negative element count");
    if (num_elements == 0) return ok();
    if (num_elements > (int64_t(1) << 38))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_affine_q4: element count too large");
    if (group_size <= 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_affine_q4: group_size must be positive");
    if (group_size > (int64_t(1) << 30)) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_affine_q4: group_size too large");
    // The format stores whole words per group (the reference kernel indexes
    // weight + group * (group_size / 8), runtime/affine_q4_dequant.cu:42-46).
    if (group_size % 8 != 0)
        return set_error(GDSLLM_ERR_UNSUPPORTED, "dequant_affine_q4: group_size must be a multiple of 8");
    if (in_dim <= 0 || in_dim % group_size != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_affine_q4: in_dim must be a positive multiple of group_size");
    if (num_elements % 8 != 0 || num_elements % group_size != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         "dequant_affine_q4: element count must be a multiple of 8 and of group_size");
    if (!weight || !scales || !biases || !dst)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_affine_q4: null pointer");
    if (reinterpret_cast<uintptr_t>(weight) % 4 != 0 || reinterpret_cast<uintptr_t>(scales) % 2 != 0 ||
        reinterpret_cast<uintptr_t>(biases) % 2 != 0 || reinterpret_cast<uintptr_t>(dst) % 2 != 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "dequant_affine_q4: misaligned pointer");
    hipStream_t s = as_stream(stream);
    if (reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
        const int64_t words = num_elements / 8;
        const int wpg = static_cast<int>(group_size / 8);
        const int64_t per_wg = kThreads * kChunksPerThread;
        const dim3 grid(static_cast<unsigned>((words + per_wg - 1) / per_wg));
        if ((wpg & (wpg - 1)) == 0)
            hipLaunchKernelGGL(dequant_affine_words<true>, grid, dim3(kThreads), 0, s,
                               static_cast<const uint32_t*>(weight), static_cast<const uint16_t*>(scales),
                               static_cast<const uint16_t*>(biases), static_cast<uint4*>(dst), words, wpg,
                               __builtin_ctz(static_cast<unsigned>(wpg)));
        else
            hipLaunchKernelGGL(dequant_affine_words<false>, grid, dim3(kThreads), 0, s,
                               static_cast<const uint32_t*>(weight), static_cast<const uint16_t*>(scales),
                               static_cast<const uint16_t*>(biases), static_cast<uint4*>(dst), words, wpg, 0);
    } else {
        hipLaunchKernelGGL(dequant_affine_elems, dim3(grid_for(num_elements)), dim3(kThreads), 0, s,
                           static_cast<const uint32_t*>(weight), static_cast<const uint16_t*>(scales),
                           static_cast<const uint16_t*>(biases), static_cast<uint16_t*>(dst), num_elements,
                           static_cast<int>(group_size));
    }
    if (int rc = check_hip(hipGetLastError(), "dequant_affine_q4 launch")) return rc;
    return ok();
}

namespace {
int embed_rows(bool q8, const void* table, const int64_t* ids, int64_t n_tokens, int64_t vocab, int64_t hidden,
               void* out, void* stream) {
    const std::string n = q8 ? "embed_q8_0" : "embed_q4_0";
    if (n_tokens < 0 || vocab < 0 || hidden < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": negative size");
    if (n_tokens == 0 || hidden == 0) return ok();
    if (!table || !ids || !out) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": null pointer");
    if (hidden % 64 != 0)
        return set_error(GDSLLM_ERR_UNSUPPORTED, n + ": hidden must be a multiple of 64, got " + std::to_string(hidden));
    if (n_tokens > 65535 || hidden > (int64_t(1) << 24))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": too many tokens (max 65535 per call) or hidden too large");
    if (reinterpret_cast<uintptr_t>(table) % 4 || reinterpret_cast<uintptr_t>(out) % 16 ||
        reinterpret_cast<uintptr_t>(ids) % 8)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, n + ": table must be 4-byte, out 16-byte, ids 8-byte aligned");
    const dim3 grid(static_cast<unsigned>((hidden / 64 + kThreads - 1) / kThreads), static_cast<unsigned>(n_tokens));
    if (q8)
        hipLaunchKernelGGL(embed_rows_pairs<true>, grid, dim3(kThreads), 0, as_stream(stream),
                           static_cast<const uint8_t*>(table), ids, vocab, hidden, static_cast<uint4*>(out));
    else
        hipLaunchKernelGGL(embed_rows_pairs<false>, grid, dim3(kThreads), 0, as_stream(stream),
                           static_cast<const uint8_t*>(table), ids, vocab, hidden, static_cast<uint4*>(out));
    if (int rc = check_hip(hipGetLastError(), (n + " launch").c_str())) return rc;
    return ok();
}
}  // namespace

extern "C" int gdsllm_embed_q4_0(const void* table, const int64_t* token_ids, int64_t n_tokens, int64_t vocab,
                                 int64_t hidden, void* out, void* stream) {
    return embed_rows(false, table, token_ids, n_tokens, vocab, hidden, out, stream);
}

extern "C" int gdsllm_embed_q8_0(const void* table, const int64_t* token_ids, int64_t n_tokens, int64_t vocab,
                                 int64_t hidden, void* out, void* stream) {
    return embed_rows(true, table, token_ids, n_tokens, vocab, hidden, out, stream);
}
