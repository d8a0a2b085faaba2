// lt_topk.h -- softmax + top-k over a router's logits in one wavefront.
// Shared by the router (last-block top-k, batched prefill top-k) and the
// expert gate/up kernel (each block routes for itself).
#pragma once

#include "lt_internal.h"

#include <math.h>

namespace lt {

// Order-preserving integer key of a (NaN-free) float: a > b <=> key(a) > key(b),
// and -0 / +0 map to the same key (they compare equal).  Keys of real values
// are >= key(-inf) = 0x007fffff, so 0 is free to mark an absent entry.
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// Softmax + top-k over n <= 64*PER logits, executed by one full wavefront
// (lane = 0..63; lane owns entries lane + 64*j).  Selection follows the
// strict '>' rule of every reference top-k (ops/moe.zig:87,
// gemma4/forward.zig:612-625): larger value first, the lower index among
// equal values; NaN logits rank as -inf.  Each of the k rounds is a
// wave-wide max over order-preserving keys -- v_max_u32 over the 16-lane
// rows (DPP rotations), the four row maxima read into scalars -- and the
// winner is the first lane holding the maximum key (ballot +
// find-first-set), whose key is then cleared.
// w[r] = exp(l - max) / sum_j exp(l_j - max); with norm, divided by the sum
// of the selected weights taken in selection order.  scores (optional):
// logits, with the selected entries replaced by their probabilities
// (routerTopKSoftmax's buffer, gemma4/forward.zig:645-668).
template <int PER>
__device__ void topk_softmax_regs(const float (&vin)[PER], int n, int k, int norm, uint32_t *ids, float *w,
                                  uint32_t (&key)[PER], int &my_i_out, float &my_p_out, int lane);

// Loads lane + 64*j (j < PER) of logits[0..n) and runs topk_softmax_regs.
template <int PER>
__device__ void topk_softmax_wave(const float *logits, int n, int k, int norm, uint32_t *ids, float *w,
                                  float *scores, int lane) {
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = lane + 64 * j;
        v[j] = idx < n ? logits[idx] : -INFINITY;
    }
    uint32_t key[PER];
    int my_i;
    float my_p;
    topk_softmax_regs<PER>(v, n, k, norm, ids, w, key, my_i, my_p, lane);
    if (scores) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int idx = lane + 64 * j;
            if (idx < n) {
                float val = logits[idx];
                if (key[j] == 0)  // selected (cleared)
                    for (int r = 0; r < k; r++)
                        if (__builtin_amdgcn_readlane(my_i, r) == idx)
                            val = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_p), r));
                scores[idx] = val;
            }
        }
    }
}

// Index of the rank-th selection (0-based) of the same rule, without the
// softmax: rank + 1 selection rounds over values in registers (vin[j] is
// entry lane + 64*j).  Used where only one slot's expert is needed.
template <int PER>
__device__ int topk_index_at(const float (&vin)[PER], int n, int rank, int lane) {
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = lane + 64 * j;
        float t = idx < n ? vin[j] : -INFINITY;
        if (t != t) t = -INFINITY;
        key[j] = idx < n ? order_key(t) : 0u;
    }
    int idx = 0;
    for (int r = 0; r <= rank; r++) {
        uint32_t mx = key[0];
#pragma unroll
        for (int j = 1; j < PER; j++) mx = max(mx, key[j]);
        mx = max(mx, dpp_u<0x128>(mx));
        mx = max(mx, dpp_u<0x124>(mx));
        mx = max(mx, dpp_u<0x122>(mx));
        mx = max(mx, dpp_u<0x121>(mx));
        const uint32_t K = max(max((uint32_t)__builtin_amdgcn_readlane(mx, 0), (uint32_t)__builtin_amdgcn_readlane(mx, 16)),
                               max((uint32_t)__builtin_amdgcn_readlane(mx, 32), (uint32_t)__builtin_amdgcn_readlane(mx, 48)));
        idx = -1;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint64_t b = __ballot(key[j] == K);
            if (idx < 0 && b) idx = 64 * j + (int)__builtin_ctzll(b);
        }
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (idx == lane + 64 * j) key[j] = 0;
    }
    return idx;
}

// The selection itself on values already in registers: vin[j] is entry
// lane + 64*j (entries >= n are ignored).  On return key[j] == 0 marks the
// selected entries, and lane r < k holds the r-th selection in my_i_out /
// my_p_out (index and weight before renormalisation); ids / w (if not
// NULL) receive the selection.
template <int PER>
__device__ void topk_softmax_regs(const float (&vin)[PER], int n, int k, int norm, uint32_t *ids, float *w,
                                  uint32_t (&key)[PER], int &my_i_out, float &my_p_out, int lane) {
    const bool first = p32_first(lane);
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = lane + 64 * j;
        float t = idx < n ? vin[j] : -INFINITY;
        if (t != t) t = -INFINITY;
        v[j] = t;
        key[j] = idx < n ? order_key(t) : 0u;
    }
    uint32_t my_key = 0;
    int my_i = 0;
    uint32_t kmax = 0;
    for (int r = 0; r < k; r++) {
        uint32_t mx = key[0];
#pragma unroll
        for (int j = 1; j < PER; j++) mx = max(mx, key[j]);
        mx = max(mx, dpp_u<0x128>(mx));
        mx = max(mx, dpp_u<0x124>(mx));
        mx = max(mx, dpp_u<0x122>(mx));
        mx = max(mx, dpp_u<0x121>(mx));
        const uint32_t K = max(max((uint32_t)__builtin_amdgcn_readlane(mx, 0), (uint32_t)__builtin_amdgcn_readlane(mx, 16)),
                               max((uint32_t)__builtin_amdgcn_readlane(mx, 32), (uint32_t)__builtin_amdgcn_readlane(mx, 48)));
        int idx = -1;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint64_t b = __ballot(key[j] == K);
            if (idx < 0 && b) idx = 64 * j + (int)__builtin_ctzll(b);
        }
        if (r == 0) kmax = K;
        if (lane == r) {
            my_key = K;
            my_i = idx;
        }
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (idx == lane + 64 * j) key[j] = 0;
    }
    const float m = key_value(kmax);  // the largest logit (NaNs read as -inf)
    float se = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++)
        if (lane + 64 * j < n) se += expf(v[j] - m);
    se += dpp<0x128>(se);
    se += dpp<0x124>(se);
    se += dpp<0x122>(se);
    se += dpp<0x121>(se);
    se += xor16(se);
    se += xor32(se, first);
    const float my_p = lane < k ? expf(key_value(my_key) - m) / se : 0.0f;
    float ps = 0.0f;  // sum of the selected weights in selection order
    if (norm)
        for (int r = 0; r < k; r++) ps = ps + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_p), r));
    if (lane < k && ids) {
        ids[lane] = (uint32_t)my_i;
        w[lane] = norm ? my_p / ps : my_p;
    }
    my_i_out = my_i;
    my_p_out = my_p;
}

}  // namespace lt
