// The reference's routing selection, shared by the host routing helpers and the device router
// so both produce the same routes from the same source.
//
// Top-k: src/pytorch_topk.cpp:8-30 calls std::nth_element(first, first + k - 1, last) over
// (value, index) pairs ordered greater-by-value, from the C++ library PyTorch was built with
// (libc++ for the reference's golden orders), and returns the first k indices in partition
// order. This is that published algorithm (libc++ <__algorithm/nth_element.h>): median of three,
// a guarded partition that tracks the pivot, the all-not-greater fallback partition, the
// already-partitioned check, and selection sort below 8 elements.
//
// Routes: pytorch_noaux_routes (src/text_endpoint.rs:4394-4473): corrected = score + bias, top 8
// of corrected, boundary check against the best rejected value (equality counts as a tie), and
// weights score_i / (pytorch_sum_eight(scores) + 1e-20) with pytorch_sum_eight
// (src/text_endpoint.rs:4382-4390) = fold(0, +) over (s0 + s4, s1 + s5, s2 + s6, s3 + s7).
#pragma once

#include <stdint.h>

#include "pw_numerics.h"

namespace pw {

// A (value, index) pair of the partition. The routing paths index at most 2^31 experts and use
// 32-bit indices; the reference's FFI keeps 64-bit ones (any count), and the algorithm below is
// the same for both.
template <class Idx>
struct TopkEntryT {
    float v;
    Idx i;
};
typedef TopkEntryT<int32_t> TopkEntry;
typedef TopkEntryT<int64_t> TopkEntry64;

template <class T>
PW_HD bool topk_greater(const T &a, const T &b) { return a.v > b.v; }

template <class T>
PW_HD void topk_swap(T &a, T &b)
{
    const T t = a;
    a = b;
    b = t;
}

template <class T>
PW_HD unsigned topk_sort3(T *x, T *y, T *z)
{
    if (!topk_greater(*y, *x)) {
        if (!topk_greater(*z, *y))
            return 0;
        topk_swap(*y, *z);
        if (topk_greater(*y, *x)) {
            topk_swap(*x, *y);
            return 2;
        }
        return 1;
    }
    if (topk_greater(*z, *y)) {
        topk_swap(*x, *z);
        return 1;
    }
    topk_swap(*x, *y);
    if (topk_greater(*z, *y)) {
        topk_swap(*y, *z);
        return 2;
    }
    return 1;
}

template <class T>
PW_HD void topk_select_sort(T *first, T *last)
{
    for (T *lm1 = last - 1; first != lm1; ++first) {
        T *best = first;
        for (T *it = first + 1; it != last; ++it)
            if (topk_greater(*it, *best))
                best = it;
        if (best != first)
            topk_swap(*first, *best);
    }
}

// The ranges of at most 7 elements nth_element finishes directly; returns false for longer ones.
template <class T>
PW_HD bool topk_small(T *first, T *last)
{
    const long len = (long)(last - first);
    if (len <= 1)
        return true;
    if (len == 2) {
        if (topk_greater(last[-1], *first))
            topk_swap(*first, last[-1]);
        return true;
    }
    if (len == 3) {
        topk_sort3(first, first + 1, last - 1);
        return true;
    }
    if (len <= 7) {
        topk_select_sort(first, last);
        return true;
    }
    return false;
}

// The partition nth_element falls back to when no element of (first, last - 1) is greater than the
// pivot and *first equals it: partitions around *first. Returns true when nth is placed; otherwise
// *next is the new start of the range.
template <class T>
PW_HD bool topk_fallback_partition(T *first, T *nth, T *last, T **next)
{
    T *i = first + 1, *j = last;
    if (!topk_greater(*first, *--j)) {
        for (;; ++i) {
            if (i == j)
                return true;
            if (topk_greater(*first, *i)) {
                topk_swap(*i, *j);
                ++i;
                break;
            }
        }
    }
    if (i == j)
        return true;
    for (;;) {
        while (!topk_greater(*first, *i))
            ++i;
        do
            --j;
        while (topk_greater(*first, *j));
        if (i >= j)
            break;
        topk_swap(*i, *j);
        ++i;
    }
    if (nth < i)
        return true;
    *next = i;
    return false;
}

template <class T>
PW_HD void nth_element_libcxx(T *first, T *nth, T *last)
{
    for (;;) {
        if (nth == last)
            return;
        if (topk_small(first, last))
            return;
        const long len = (long)(last - first);
        T *m = first + len / 2, *lm1 = last - 1;
        unsigned swaps = topk_sort3(first, m, lm1);
        T *i = first, *j = lm1;
        if (!topk_greater(*i, *m)) {
            bool guard = false;
            while (!(i == --j)) {
                if (topk_greater(*j, *m)) {
                    guard = true;
                    break;
                }
            }
            if (guard) {
                topk_swap(*i, *j);
                ++swaps;
            } else {
                T *next;
                if (topk_fallback_partition(first, nth, last, &next))
                    return;
                first = next;
                continue;
            }
        }
        ++i;
        if (i < j) {
            for (;;) {
                while (topk_greater(*i, *m))
                    ++i;
                do
                    --j;
                while (!topk_greater(*j, *m));
                if (i >= j)
                    break;
                topk_swap(*i, *j);
                ++swaps;
                if (m == i)
                    m = j;
                ++i;
            }
        }
        if (i != m && topk_greater(*m, *i)) {
            topk_swap(*i, *m);
            ++swaps;
        }
        if (nth == i)
            return;
        if (swaps == 0) {
            T *a = nth < i ? first : i, *end = nth < i ? i : last, *prev = a;
            bool sorted = true;
            while (++a != end) {
                if (topk_greater(*a, *prev)) {
                    sorted = false;
                    break;
                }
                prev = a;
            }
            if (sorted)
                return;
        }
        if (nth < i)
            last = i;
        else
            first = i + 1;
    }
}

// Outcome of one routed row.
enum RouteStatus : int { ROUTE_OK = 0, ROUTE_NONFINITE = 1, ROUTE_TOPK = 2, ROUTE_WEIGHTS = 3 };

// The end of one row after the top-k partition: sel8[0..8) holds the selected (corrected, id)
// entries in partition order, chosen[k] the uncorrected score of sel8[k]'s expert, and `rejected`
// is the largest corrected value of the rest. Checks the boundary (equality counts as a tie) and
// writes selected[8], weights[8].
PW_HD int noaux_finish_row8(const TopkEntry *sel8, const float *chosen, float rejected, uint32_t *selected,
                            float *weights, bool *tie)
{
    constexpr uint32_t K = 8;
    uint32_t sel[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        sel[k] = (uint32_t)sel8[k].i;
#pragma unroll
        for (uint32_t j = 0; j < k; ++j)
            if (sel[j] == sel[k])
                return ROUTE_TOPK;
    }
    float boundary = sel8[0].v;
#pragma unroll
    for (uint32_t k = 1; k < K; ++k)
        boundary = sel8[k].v < boundary ? sel8[k].v : boundary;
    if (!finite_f32_bits(boundary) || boundary < rejected)
        return ROUTE_TOPK;
    *tie = boundary == rejected;
    const float lanes[4] = {chosen[0] + chosen[4], chosen[1] + chosen[5], chosen[2] + chosen[6],
                            chosen[3] + chosen[7]};
    float sum = 0.0f;
#pragma unroll
    for (uint32_t l = 0; l < 4; ++l)
        sum = sum + lanes[l];
    const float denominator = sum + 1.0e-20f;
    float wsum = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        const float w = chosen[k] / denominator;
        if (!finite_f32_bits(w) || w < 0.0f)
            return ROUTE_WEIGHTS;
        weights[k] = w;
        selected[k] = sel[k];
        wsum += w;
    }
    const float dev = wsum - 1.0f;
    if ((dev < 0.0f ? -dev : dev) > 1.0e-6f)
        return ROUTE_WEIGHTS;
    return ROUTE_OK;
}

// The same from the full scores row and the partitioned entries.
PW_HD int noaux_finish_row(const float *scores, const TopkEntry *scratch, float rejected, uint32_t *selected,
                           float *weights, bool *tie)
{
    float chosen[8];
    for (uint32_t k = 0; k < 8; ++k)
        chosen[k] = scores[scratch[k].i];
    return noaux_finish_row8(scratch, chosen, rejected, selected, weights, tie);
}

// One row of pytorch_noaux_routes: scores [experts] (sigmoid outputs), bias [experts] ->
// selected[8], weights[8]; *tie = the boundary value equals the best rejected value. `scratch`
// holds `experts` entries. Returns a RouteStatus.
PW_HD int noaux_route_row(const float *scores, const float *bias, uint32_t experts, TopkEntry *scratch,
                          uint32_t *selected, float *weights, bool *tie)
{
    *tie = false;
    for (uint32_t e = 0; e < experts; ++e) {
        if (!finite_f32_bits(scores[e]) || !finite_f32_bits(bias[e]))
            return ROUTE_NONFINITE;
        scratch[e].v = scores[e] + bias[e];
        scratch[e].i = (int32_t)e;
    }
    nth_element_libcxx(scratch, scratch + 7, scratch + experts);
    float rejected = -__builtin_inff();
    for (uint32_t k = 8; k < experts; ++k)
        rejected = scratch[k].v > rejected ? scratch[k].v : rejected;
    return noaux_finish_row(scores, scratch, rejected, selected, weights, tie);
}

}  // namespace pw
