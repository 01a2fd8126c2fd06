// Shared helpers for the gfx950 kernels and the C ABI around them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "gdsllm_amd.h"

namespace gdsllm {

// ----------------------------------------------------------------- host side

// Records `msg` as this thread's last error and returns `code`.
int set_error(int code, const std::string& msg);
// Clears the thread's last error and returns GDSLLM_OK.
int ok();
// Checks the result of a HIP call or launch; on failure records
// "<what>: <hip error string>" and returns GDSLLM_ERR_HIP.
int check_hip(hipError_t err, const char* what);
// Number of compute units of the current device (cached per device).
int cu_count();
// Maximum dynamic LDS bytes a workgroup may use on the current device.
int max_lds_bytes();
// Allows `fn` to launch with `lds` dynamic LDS bytes (above the 64 KiB default).
int prepare_lds(const void* fn, size_t lds);
// Workgroups of `threads` threads of kernel `fn` with `lds` dynamic LDS bytes
// that fit on one compute unit (at least 1; cached).
int blocks_per_cu(const void* fn, size_t lds, int threads);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Q4_0 prefill GEMM for in_dim % 32 == 0 off the split-K grid (gemm.hip);
// arguments already validated.
int dequant_gemm_q4_0_blockwise(const void* weight, const void* x, void* y, int M, int K, int T, int64_t ldx,
                                int64_t ldy, hipStream_t stream);

// ---------------------------------------------------------------- device side

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming (non-temporal) global load.
__device__ __forceinline__ uint4 load_nt16(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(bits16)));
}
// Returns `v` as a materialized fp32 register value.  Without it the compiler
// folds "fp32 multiply(-add), then convert to fp16" into one v_fma_mixlo_f16,
// which rounds once (the reference rounds to fp32 first) and adds +0 to a
// plain product (turning an IEEE -0 into +0).  Bit-exact paths need both
// roundings and the sign of zero, so they pass through this barrier.
__device__ __forceinline__ float fp32_rounded(float v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint16_t f2h_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<half_t>(v));
}
__device__ __forceinline__ uint32_t pack_h2(half_t lo, half_t hi) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
}

// fp32 += a.lo*b.lo + a.hi*b.hi with a, b packed fp16 pairs (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                  __builtin_bit_cast(half2_t, b), c, false);
}

// Bytes [2, 6) of the little-endian pair (lo, hi): re-aligns a dword stream
// that starts on a 2-byte boundary.
__device__ __forceinline__ uint32_t align2(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// Two fp16 weights from two 4-bit fields of `v`.  Fields at bits [0,4) and
// [16,20) become 1024+q (exponent 2^10, ulp 1); fields at bits [4,8) and
// [20,24) become 64+q (exponent 2^6, ulp 1/16 so bits 4..7 weigh 1).
__device__ __forceinline__ uint32_t nib_lo_pair(uint32_t v) {
    return (v & 0x000F000Fu) | 0x64006400u;
}
__device__ __forceinline__ uint32_t nib_hi_pair(uint32_t v) {
    return (v & 0x00F000F0u) | 0x54005400u;
}

// The same two nibble-pair conversions as single v_and_or_b32 instructions.
// gfx9 VOP3 encodings take no literal constants, so written with literals the
// compiler splits each into v_and + v_or; here the masks live in SGPRs and the
// exponent bits in VGPRs, made opaque once per kernel so they are not
// rematerialized at every use.
struct NibUnpack {
    uint32_t mask_lo, mask_hi;  // SGPR
    uint32_t bits_lo, bits_hi;  // VGPR
    __device__ __forceinline__ NibUnpack() : mask_lo(0x000F000Fu), mask_hi(0x00F000F0u), bits_lo(0x64006400u), bits_hi(0x54005400u) {
        asm volatile("" : "+s"(mask_lo), "+s"(mask_hi), "+v"(bits_lo), "+v"(bits_hi));
    }
    __device__ __forceinline__ uint32_t lo(uint32_t v) const {
        uint32_t r;
        asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask_lo), "v"(bits_lo));
        return r;
    }
    __device__ __forceinline__ uint32_t hi(uint32_t v) const {
        uint32_t r;
        asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask_hi), "v"(bits_hi));
        return r;
    }
    // The same conversions written in C on the opaque registers (the compiler
    // still forms one v_and_or_b32 each).  Required where the result feeds an
    // MFMA directly: the compiler inserts the VALU-write -> MFMA-read wait
    // states only after instructions it can see, so an MFMA operand written by
    // the asm forms above may be read before the write has landed.
    __device__ __forceinline__ uint32_t lo_c(uint32_t v) const { return (v & mask_lo) | bits_lo; }
    __device__ __forceinline__ uint32_t hi_c(uint32_t v) const { return (v & mask_hi) | bits_hi; }
};

// v read from another lane of the same 16-lane DPP row (VALU data movement).
template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of each DPP row (lanes 16r .. 16r+15), every lane of
// the row receiving the total: quad xor 1, quad xor 2, then the half-row
// mirror (i <-> 7-i) and the row mirror (i <-> 15-i).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_read<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_read<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_read<0x141>(v);  // row_half_mirror
    v += dpp_read<0x140>(v);  // row_mirror
    return v;
}
// a + b after swapping lanes 32..63 of a with lanes 0..31 of b
// (v_permlane32_swap_b32): lanes 0..31 get a[l] + a[l+32], lanes 32..63 get
// b[l-32] + b[l].  swap16 does the same for 16-lane halves within each 32-lane
// half.  Written as inline asm (with the swap-to-swap wait states) because
// this toolchain's builtins return both swapped values in one register.
__device__ __forceinline__ float swap_sum32(float a, float b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ __forceinline__ float swap_sum16(float a, float b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return a + b;
}
// The swap itself: afterwards a = [a lanes 0..31, b lanes 0..31] and
// b = [a lanes 32..63, b lanes 32..63].
__device__ __forceinline__ void swap32(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// SwiGLU input h = silu(gate) * up with torch semantics on fp16 tensors: the
// gate and up sums are fp16 values; silu is computed in fp32 and rounded to
// fp16, then the fp16 product is computed in fp32 and rounded once.
__device__ __forceinline__ uint16_t silu_mul_h(float g, float u) {
    const float gh = h2f(f2h_bits(g));
    const float sg = h2f(f2h_bits(gh / (1.0f + expf(-gh))));
    return f2h_bits(sg * h2f(f2h_bits(u)));
}

// Sum over groups of `width` lanes (power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WIDTH);
    return v;
}

// Row dot products of fp16 weights (gemv_f16 and everything that must give
// its bits) in one fixed order: the row's 512-column chunks are dealt to four
// parts, chunk c to part c % 4; within a part lane l takes 8 weights of each
// of its chunks, in chunk order, with v_dot2 into fp32, then the part is
// summed over the wave (group_sum<64>); the row is ((p0 + p1) + p2) + p3.
// gemv_f16 runs the four parts on four waves of a workgroup.

// This lane's sum over the chunks of part `part` of row w (K % 8 == 0, w and
// x 16-byte aligned).
__device__ __forceinline__ float f16_part_lane(const uint16_t* __restrict__ w, const uint16_t* __restrict__ x, int K,
                                               int part, int lane) {
    float acc = 0.f;
    for (int c = 8 * lane + 512 * part; c < K; c += 2048) {
        const uint4 wv = *reinterpret_cast<const uint4*>(w + c);
        const uint4 xv = *reinterpret_cast<const uint4*>(x + c);
        acc = dot2(wv.x, xv.x, acc);
        acc = dot2(wv.y, xv.y, acc);
        acc = dot2(wv.z, xv.z, acc);
        acc = dot2(wv.w, xv.w, acc);
    }
    return acc;
}

// One fp16 row dot x by one wave, the four parts in turn: the same inputs give
// the same bits as gdsllm_gemv_f16.
__device__ __forceinline__ float f16_row_dot(const uint16_t* __restrict__ w, const uint16_t* __restrict__ x, int K,
                                             int lane) {
    float p[4];
#pragma unroll
    for (int part = 0; part < 4; ++part) p[part] = group_sum<64>(f16_part_lane(w, x, K, part, lane));
    return ((p[0] + p[1]) + p[2]) + p[3];
}

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4,
// non-temporal): lane l's bytes land at lds + 16*l.  `lds` must be the same for
// every lane of the wave (it goes to M0).  The transfer is tracked by vmcnt
// like a load; the data is readable from LDS once a vmcnt wait covers it.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(lds), 16, 0,
                                     /*nt*/ 2);
}

// The same with the default cache policy: for data many workgroups read (the
// activation vector), which should stay in L2 after its first miss.
__device__ __forceinline__ void dma16_cached(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(lds), 16, 0, 0);
}

// Waits until at most N vector-memory operations of this wave are in flight
// (s_waitcnt vmcnt(N); expcnt and lgkmcnt untouched).  Vector memory loads
// retire in issue order, so this waits for all but the last N issued.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
    asm volatile("" ::: "memory");
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One LDS-DMA transfer of 16 (4) bytes per lane from base + voff[lane] to
// lds + 16l (4l); base and lds are wave-uniform (lds goes to M0).  Written as
// inline asm, the transfers are invisible to the compiler's counters: it
// neither waits for them before its own LDS accesses nor counts them, so a
// kernel using them waits with wait_vmcnt_asm and keeps every other vector
// memory operation out of the windows it counts.
__device__ __forceinline__ void dma16_asm(uint32_t voff, const void* base, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "m0");
}
__device__ __forceinline__ void dma4_asm(uint32_t voff, const void* base, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void wait_vmcnt_asm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS accesses written as instructions the compiler does not analyse.  The
// compiler orders every LDS access it sees after all in-flight LDS DMA
// transfers it cannot prove disjoint from it, i.e. it waits for every
// transfer; these let a kernel touch a region no transfer writes (prepared
// x, a dequantized tile) while transfers into other buffers are in flight.
// Each read helper issues its reads and "s_waitcnt lgkmcnt(0)" in ONE asm
// statement: the results exist only when the statement ends, so no copy the
// register allocator places after it can see a register the read has not
// yet filled (a separate wait statement cannot rule such copies out).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}
__device__ __forceinline__ void lds_write16_raw(uint32_t addr, u32x4_t v) {
    asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write4_raw(uint32_t addr, uint32_t v) {
    asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
// 16 bytes at addr (16-byte aligned).
__device__ __forceinline__ u32x4_t lds_read16_sync(uint32_t addr) {
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
    return v;
}
// 16 bytes at each of addr + STRIDE * i, i < 4 (16-byte aligned).
template <int STRIDE>
__device__ __forceinline__ void lds_read16x4_sync(uint32_t addr, u32x4_t (&v)[4]) {
    static_assert(STRIDE % 16 == 0 && 3 * STRIDE < 65536, "ds offset range");
    asm volatile(
        "ds_read_b128 %0, %4\n\t"
        "ds_read_b128 %1, %4 offset:%5\n\t"
        "ds_read_b128 %2, %4 offset:%6\n\t"
        "ds_read_b128 %3, %4 offset:%7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
        : "v"(addr), "i"(STRIDE), "i"(2 * STRIDE), "i"(3 * STRIDE));
}
// 16 bytes at each of addr + 1024 * i, i < 8 (16-byte aligned).
__device__ __forceinline__ void lds_read16x8_sync(uint32_t addr, u32x4_t (&v)[8]) {
    asm volatile(
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %8 offset:1024\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\t"
        "ds_read_b128 %3, %8 offset:3072\n\t"
        "ds_read_b128 %4, %8 offset:4096\n\t"
        "ds_read_b128 %5, %8 offset:5120\n\t"
        "ds_read_b128 %6, %8 offset:6144\n\t"
        "ds_read_b128 %7, %8 offset:7168\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
        : "v"(addr));
}
// 24 bytes at addr (only 4-byte aligned), as three dword pairs.
__device__ __forceinline__ void lds_read4x6_sync(uint32_t addr, uint64_t (&v)[3]) {
    asm volatile(
        "ds_read2_b32 %0, %3 offset1:1\n\t"
        "ds_read2_b32 %1, %3 offset0:2 offset1:3\n\t"
        "ds_read2_b32 %2, %3 offset0:4 offset1:5\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2])
        : "v"(addr));
}
// Workgroup barrier for LDS data only: this wave's LDS requests complete, then
// s_barrier.  Unlike __syncthreads it does not wait for outstanding global
// loads or LDS DMA transfers.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Orders this wave's earlier LDS writes before its later LDS reads.  LDS
// requests of one wavefront are served in issue order; the waitcnt and the
// memory clobber keep the compiler from moving reads above the writes.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

}  // namespace gdsllm
