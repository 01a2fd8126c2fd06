// Top-k expert selection by one wave, shared by route_topk (route.hip) and
// the routed MoE decode step (affine.hip), so both give the same picks and
// weights bit for bit.
//
// The reference takes torch.topk of the router logits and a float32 softmax of
// the k values cast back to fp16 (runtime/qwen_moe.py:405-412).  Here each
// logit becomes a pick word (an order key above an inverted index), k rounds
// of a wave-wide max take the picks in descending order, and the softmax sums
// exp(l - max) in fp32 in pick order.
#pragma once

#include "common.h"

namespace gdsllm {

// Pick word of logit e: a 16-bit order key of the fp16 value above a 16-bit
// inverted index, so the largest word is the largest logit and, among equal
// logits, the lowest index.  The key is monotone in the value (negative
// encodings inverted, positive ones offset above them), -0 and +0 share a key
// (torch.topk sees them as equal) and every NaN ranks above +inf.  The
// smallest key, -inf's, is 0x03FF, so a word of 0 never occurs: it marks a
// logit already taken (or a lane slot past the last expert).
__device__ __forceinline__ uint32_t pick_word(uint32_t h, int e) {
    const uint32_t mag = h & 0x7FFFu;
    uint32_t key = (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
    key = mag == 0 ? 0x8000u : key;         // +-0
    key = mag > 0x7C00u ? 0xFFFFu : key;    // NaN
    return (key << 16) | (0xFFFFu - static_cast<uint32_t>(e));
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// Maximum over the wave, returned wave-uniform: DPP within each 16-lane row
// (quad xor 1, quad xor 2, half-row mirror, row mirror), then the four row
// maxima through readlane.
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    v = max(v, dpp_u32<0x140>(v));
    const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return max(max(r0, r1), max(r2, r3));
}

// The k picks of the words spread over the wave (NPL per lane, in any
// arrangement): each round's pick is wave-uniform, its owner clears it, and
// lane i keeps pick i (expert index my_idx, order key my_key); top_key is the
// largest key.  Only the selection is serial.
template <int NPL>
__device__ __forceinline__ void topk_select(uint32_t (&word)[NPL], int k, int lane, int& my_idx, uint32_t& my_key,
                                            uint32_t& top_key) {
    my_idx = 0;
    my_key = 0;
    top_key = 0;
    for (int i = 0; i < k; ++i) {
        uint32_t best = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j) best = word[j] > best ? word[j] : best;
        best = wave_max(best);
#pragma unroll
        for (int j = 0; j < NPL; ++j) word[j] = word[j] == best ? 0u : word[j];
        if (i == 0) top_key = best >> 16;
        if (lane == i) {
            my_idx = static_cast<int>(0xFFFFu - (best & 0xFFFFu));
            my_key = best >> 16;
        }
    }
}

// fp16 softmax weight of this lane's pick (lanes < k): each lane decodes its
// pick's value (+-0 -> +0, NaN -> NaN, both softmax-neutral) and takes
// exp(l - max) itself, and the exponentials are summed in pick order.
__device__ __forceinline__ uint16_t topk_weight(uint32_t my_key, uint32_t top_key, int k, int lane) {
    auto key_value = [](uint32_t key) {
        return key == 0xFFFFu ? __builtin_nanf("") : h2f((key & 0x8000u) ? (key & 0x7FFFu) : (~key & 0xFFFFu));
    };
    const float m = key_value(top_key);
    const float my_ex = lane < k ? expf(fp32_rounded(key_value(my_key) - m)) : 0.f;
    float sum = 0.f;
    for (int i = 0; i < k; ++i)
        sum = fp32_rounded(sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_ex), i)));
    return f2h_bits(fp32_rounded(my_ex / sum));
}

}  // namespace gdsllm
