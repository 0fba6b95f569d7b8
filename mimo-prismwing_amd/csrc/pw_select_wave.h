// libc++ nth_element over a row of (value, index) entries held in one wave's registers, for the
// device router's top-8 (pytorch_topk.cpp:8-30 calls std::nth_element(first, first + k - 1, last)
// over (value, index) pairs ordered greater-by-value; pw_topk.h restates that algorithm).
//
// Position p = 64 c + lane of the row sits in register c of that lane (NC registers cover 64 NC
// positions). Each partition step of the serial algorithm is formed from wave ballots instead of
// element-by-element scans:
//   - reads and writes of single positions (median of three, the guard swap, the pivot fix-up,
//     ranges of at most seven entries) are lane reads and predicated register writes;
//   - the Hoare partition around the pivot value pv: with A the ascending positions in [first + 1,
//     j0] whose value is not greater than pv and B the descending positions in [first, j0 - 1]
//     whose value is, the serial loop swaps A[t] with B[t] exactly while A[t] < B[t] (t < T),
//     stops at i = min(A[T], B[T - 1]) (A[0] when T = 0) and moves the pivot from A[r] to B[r]
//     when r < T. A position's rank in A is a prefix popcount of the A masks; A[t] < B[t] holds
//     exactly when more than t positions above A[t] belong to B. The T swapped pairs exchange
//     their entries through the wave's LDS buffer in one write and one read.
// The rare fallback partition (no position of (first, last - 1) greater than a pivot equal to
// *first) runs the serial code on one lane over an LDS copy of the row.
//
// Positions are read and written one lane at a time under wave-uniform branches, the partition
// masks and their counts are wave-uniform (scalar) values, and each pass touches only the registers
// its range covers; the range holding nth = 7 shrinks towards the front, so the later passes work
// on register 0 alone.
//
// The algorithm is written against a wave policy W (lane id, ballot, count of set bits below the
// lane, lane read and write, shift by one lane, wave maximum, LDS ordering, and a progress mark
// that timing builds may record), so the device router and a CPU build that emulates a 64-lane wave
// with threads run the same source.
#pragma once

#include <stdint.h>

#include "pw_topk.h"

#if defined(__HIPCC__)
#define PW_WAVE __device__ __forceinline__
#else
#define PW_WAVE inline
#endif

namespace pw {

template <int NC>
struct WaveRow {
    float v[NC];
    int32_t id[NC];
};

PW_WAVE uint32_t popc64(uint64_t m) { return (uint32_t)__builtin_popcountll(m); }

// Bits of register c's lanes at positions [lo, hi] (inclusive; lo and hi wave-uniform, scalar work).
PW_WAVE uint64_t range_bits(int c, uint32_t lo, uint32_t hi)
{
    const int32_t b = 64 * c;
    const int32_t a0 = (int32_t)lo - b < 0 ? 0 : (int32_t)lo - b;
    const int32_t a1 = (int32_t)hi - b > 63 ? 63 : (int32_t)hi - b;
    if (lo > hi || a0 > a1)
        return 0;
    const uint64_t upto = a1 == 63 ? ~0ull : ((2ull << a1) - 1);
    return upto & ~((1ull << a0) - 1);
}

// The entry at position p (p wave-uniform, in registers 0..NCA-1): a uniform branch to p's register
// and one lane read per field.
template <int NCA, int NC, class W>
PW_WAVE TopkEntry wave_get(W &w, const WaveRow<NC> &a, uint32_t p)
{
    const uint32_t k = p >> 6, l = p & 63;
    TopkEntry e{0.f, 0};
#pragma unroll
    for (int c = 0; c < NCA; ++c)
        if (k == (uint32_t)c)
            e = TopkEntry{w.readlane(a.v[c], l), w.readlane(a.id[c], l)};
    return e;
}

// Writes e at position p (p and e wave-uniform). Every register 0..NCA-1 is assigned (unchanged
// but in p's lane): stores under per-register branches may be merged into one store through a
// selected address, which keeps the row in private memory.
template <int NCA, int NC, class W>
PW_WAVE void wave_set(W &w, WaveRow<NC> &a, uint32_t p, TopkEntry e)
{
    const uint32_t k = p >> 6, l = p & 63;
#pragma unroll
    for (int c = 0; c < NCA; ++c) {
        const uint32_t lc = k == (uint32_t)c ? l : 64u;  // lane 64: no lane
        a.v[c] = w.writelane(a.v[c], e.v, lc);
        a.id[c] = w.writelane(a.id[c], e.i, lc);
    }
}

template <int NCA, int NC, class W>
PW_WAVE unsigned wave_sort3(W &w, WaveRow<NC> &a, uint32_t x, uint32_t y, uint32_t z)
{
    TopkEntry ex = wave_get<NCA>(w, a, x), ey = wave_get<NCA>(w, a, y), ez = wave_get<NCA>(w, a, z);
    const unsigned swaps = topk_sort3(&ex, &ey, &ez);
    if (swaps) {
        wave_set<NCA>(w, a, x, ex);
        wave_set<NCA>(w, a, y, ey);
        wave_set<NCA>(w, a, z, ez);
    }
    return swaps;
}

// topk_small on the len <= 7 entries at [first, first + len), with static indices throughout
template <int NC, class W>
PW_WAVE void wave_small(W &w, WaveRow<NC> &a, uint32_t first, uint32_t len)
{
    if (len <= 1)
        return;
    TopkEntry e[7];
#pragma unroll
    for (uint32_t i = 0; i < 7; ++i)
        e[i] = i < len ? wave_get<NC>(w, a, first + i) : TopkEntry{0.f, 0};
    if (len == 2) {
        if (topk_greater(e[1], e[0]))
            topk_swap(e[0], e[1]);
    } else if (len == 3) {
        topk_sort3(&e[0], &e[1], &e[2]);
    } else {
        // selection sort: the first greatest entry of [s, len) goes to s
#pragma unroll
        for (uint32_t s = 0; s < 6; ++s) {
            if (s + 1 >= len)
                break;
            uint32_t best = s;
            TopkEntry bv = e[s];
#pragma unroll
            for (uint32_t b = s + 1; b < 7; ++b)
                if (b < len && topk_greater(e[b], bv)) {
                    best = b;
                    bv = e[b];
                }
            if (best != s) {
                const TopkEntry t = e[s];
                e[s] = bv;
#pragma unroll
                for (uint32_t b = s + 1; b < 7; ++b)
                    if (b == best)
                        e[b] = t;
            }
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < 7; ++i)
        if (i < len)
            wave_set<NC>(w, a, first + i, e[i]);
}

// copies positions [0, min(n, 64 NCA)) of the row into lds / back from it
template <int NCA, int NC, class W>
PW_WAVE void wave_to_lds(W &w, const WaveRow<NC> &a, uint32_t n, TopkEntry *lds)
{
#pragma unroll
    for (int c = 0; c < NCA; ++c) {
        const uint32_t p = 64 * c + w.lane();
        if (p < n)
            lds[p] = TopkEntry{a.v[c], a.id[c]};
    }
    w.lds_sync();
}

template <int NCA, int NC, class W>
PW_WAVE void wave_from_lds(W &w, WaveRow<NC> &a, uint32_t n, const TopkEntry *lds)
{
    w.lds_sync();
#pragma unroll
    for (int c = 0; c < NCA; ++c) {
        const uint32_t p = 64 * c + w.lane();
        if (p < n) {
            const TopkEntry e = lds[p];
            a.v[c] = e.v;
            a.id[c] = e.i;
        }
    }
    w.lds_sync();
}

// The position whose rank is r among the flagged positions: the register holding rank r from the
// uniform counts, then the lane from one ballot.
template <int NCA, class W>
PW_WAVE int32_t rank_pos(W &w, const bool (&in)[NCA], const uint32_t (&rank)[NCA], const uint32_t (&base)[NCA],
                         const uint64_t (&mask)[NCA], uint32_t r)
{
    int32_t pos = -1;
#pragma unroll
    for (int c = 0; c < NCA; ++c)
        if (r >= base[c] && r < base[c] + popc64(mask[c])) {
            const uint64_t mk = w.ballot(in[c] && rank[c] == r);
            pos = 64 * c + __builtin_ctzll(mk);
        }
    return pos;
}

// One pass of nth_element_libcxx's loop over [first, last) with len > 7 and last <= 64 NCA, so the
// range lies in registers 0..NCA-1 and no other register is touched. Returns true when nth is in
// place; otherwise first / last hold the next range.
template <int NCA, int NC, class W>
PW_WAVE bool wave_level(W &w, WaveRow<NC> &a, uint32_t nth, uint32_t n, TopkEntry *lds, uint32_t &first,
                        uint32_t &last)
{
    const uint32_t lane = w.lane();
    const uint32_t len = last - first;
    uint32_t m = first + len / 2;
    const uint32_t lm1 = last - 1;
    unsigned swaps = wave_sort3<NCA>(w, a, first, m, lm1);
    const float pv = wave_get<NCA>(w, a, m).v;
    uint32_t j0 = lm1;
    if (!(wave_get<NCA>(w, a, first).v > pv)) {
        // guard: the highest position in (first, lm1) greater than the pivot
        int32_t q = -1;
#pragma unroll
        for (int c = NCA - 1; c >= 0; --c) {
            const uint64_t mk = w.ballot(a.v[c] > pv) & range_bits(c, first + 1, lm1 - 1);
            if (q < 0 && mk)
                q = 64 * c + 63 - __builtin_clzll(mk);
        }
        if (q >= 0) {
            const TopkEntry ef = wave_get<NCA>(w, a, first), eq = wave_get<NCA>(w, a, (uint32_t)q);
            wave_set<NCA>(w, a, first, eq);
            wave_set<NCA>(w, a, (uint32_t)q, ef);
            ++swaps;
            j0 = (uint32_t)q;
        } else {
            // the all-not-greater fallback, serially on lane 0 over an LDS copy of the range
            wave_to_lds<NCA>(w, a, n, lds);
            uint32_t next = 0, done = 0;
            if (lane == 0) {
                TopkEntry *nx = nullptr;
                done = topk_fallback_partition(lds + first, lds + nth, lds + last, &nx) ? 1u : 0u;
                next = done ? 0u : (uint32_t)(nx - lds);
            }
            done = w.readlane(done, 0u);
            next = w.readlane(next, 0u);
            wave_from_lds<NCA>(w, a, n, lds);
            if (done)
                return true;
            first = next;
            return false;
        }
    }
    uint32_t i = first + 1;
    if (i < j0) {
        w.mark();
        // A: positions of [i0, j0] not greater than pv (ascending); B: positions of [first, j0 - 1]
        // greater than pv (descending). Masks and their counts are wave-uniform (scalar work).
        const uint32_t i0 = i;
        uint64_t mA[NCA], mB[NCA];
        uint32_t baseA[NCA], baseB[NCA], cntB[NCA];
        uint32_t nA = 0;
#pragma unroll
        for (int c = 0; c < NCA; ++c) {
            const uint64_t gt = w.ballot(a.v[c] > pv);
            mA[c] = range_bits(c, i0, j0) & ~gt;
            mB[c] = range_bits(c, first, j0 - 1) & gt;
            baseA[c] = nA;
            nA += popc64(mA[c]);
            cntB[c] = popc64(mB[c]);
        }
        uint32_t acc = 0;
#pragma unroll
        for (int c = NCA - 1; c >= 0; --c) {
            baseB[c] = acc;  // B positions in the registers above c
            acc += cntB[c];
        }
        // per lane: rank in A (A positions below), B positions above (a B lane's rank in B)
        bool inA[NCA], inB[NCA];
        uint32_t rankA[NCA], upB[NCA];
        uint32_t T = 0;
#pragma unroll
        for (int c = 0; c < NCA; ++c) {
            inA[c] = (mA[c] >> lane) & 1u;
            inB[c] = (mB[c] >> lane) & 1u;
            rankA[c] = baseA[c] + w.below(mA[c]);
            upB[c] = baseB[c] + cntB[c] - w.below(mB[c]) - (inB[c] ? 1u : 0u);
            // A[t] < B[t] exactly when more than t positions of B lie above A[t]
            T += popc64(w.ballot(inA[c] && rankA[c] < upB[c]));
        }
        if (T == 0) {
            int32_t pos = -1;  // A[0]: the lowest A position
#pragma unroll
            for (int c = 0; c < NCA; ++c)
                if (pos < 0 && mA[c])
                    pos = 64 * c + __builtin_ctzll(mA[c]);
            i = (uint32_t)pos;
        } else {
            const int32_t pa = T < nA ? rank_pos<NCA>(w, inA, rankA, baseA, mA, T) : -1;
            const int32_t pb = rank_pos<NCA>(w, inB, upB, baseB, mB, T - 1);
            i = (pa >= 0 && pa < pb) ? (uint32_t)pa : (uint32_t)pb;
        }
        if (m >= i0 && m <= j0) {
            // the pivot's rank in A, from the masks
            const uint32_t k = m >> 6;
            uint32_t rm = 0;
#pragma unroll
            for (int c = 0; c < NCA; ++c)
                if (k == (uint32_t)c)
                    rm = baseA[c] + popc64(mA[c] & ((1ull << (m & 63)) - 1));
            if (rm < T)
                m = (uint32_t)rank_pos<NCA>(w, inB, upB, baseB, mB, rm);
        }
        if (T) {
            // pair t: A[t]'s entry to lds[t], B[t]'s to lds[32 NC + t]; then each takes the other
            constexpr uint32_t HALF = 32 * NC;
#pragma unroll
            for (int c = 0; c < NCA; ++c) {
                if (inA[c] && rankA[c] < T)
                    lds[rankA[c]] = TopkEntry{a.v[c], a.id[c]};
                else if (inB[c] && upB[c] < T)
                    lds[HALF + upB[c]] = TopkEntry{a.v[c], a.id[c]};
            }
            w.lds_sync();
#pragma unroll
            for (int c = 0; c < NCA; ++c) {
                if (inA[c] && rankA[c] < T) {
                    const TopkEntry e = lds[HALF + rankA[c]];
                    a.v[c] = e.v;
                    a.id[c] = e.i;
                } else if (inB[c] && upB[c] < T) {
                    const TopkEntry e = lds[upB[c]];
                    a.v[c] = e.v;
                    a.id[c] = e.i;
                }
            }
            w.lds_sync();
            swaps += T;
        }
    }
    if (i != m) {
        const TopkEntry ei = wave_get<NCA>(w, a, i), em = wave_get<NCA>(w, a, m);
        if (em.v > ei.v) {
            wave_set<NCA>(w, a, i, em);
            wave_set<NCA>(w, a, m, ei);
            ++swaps;
        }
    }
    if (nth == i)
        return true;
    if (swaps == 0) {
        // already partitioned: is the side holding nth non-increasing?
        const uint32_t lo = nth < i ? first : i, end = nth < i ? i : last;
        bool up = false;
#pragma unroll
        for (int c = 0; c < NCA; ++c) {
            const uint32_t p = 64 * c + lane;
            float prev = w.shift_up1(a.v[c]);
            if (c > 0) {
                const float top = w.readlane(a.v[c > 0 ? c - 1 : 0], 63u);
                prev = lane == 0 ? top : prev;
            }
            up |= p > lo && p < end && a.v[c] > prev;
        }
        if (w.ballot(up) == 0)
            return true;
    }
    if (nth < i)
        last = i;
    else
        first = i + 1;
    return false;
}

// nth_element_libcxx(a, a + nth, a + n) on the wave's row; lds holds 64 NC entries for this wave.
// Each pass works on the registers its range covers (nth = 7 keeps the range near the front, so
// after the first passes it fits in register 0).
template <int NC, class W>
PW_WAVE void nth_element_wave_regs(W &w, WaveRow<NC> &a, uint32_t nth, uint32_t n, TopkEntry *lds)
{
    uint32_t first = 0, last = n;
    for (;;) {
        w.mark();
        if (nth == last)
            return;
        const uint32_t len = last - first;
        if (len <= 7) {
            wave_small(w, a, first, len);
            w.mark();
            return;
        }
        bool done;
        if (last <= 64)
            done = wave_level<1>(w, a, nth, n, lds, first, last);
        else if (NC >= 2 && last <= 128)
            done = wave_level<(NC >= 2 ? 2 : NC)>(w, a, nth, n, lds, first, last);
        else if (NC >= 4 && last <= 256)
            done = wave_level<(NC >= 4 ? 4 : NC)>(w, a, nth, n, lds, first, last);
        else if (NC >= 8 && last <= 512)
            done = wave_level<(NC >= 8 ? 8 : NC)>(w, a, nth, n, lds, first, last);
        else
            done = wave_level<NC>(w, a, nth, n, lds, first, last);
        if (done)
            return;
    }
}

// The row's scores and bias at positions e = 64 c + lane, read by every lane (positions past E,
// E >= 1, reread position E - 1, so no load sits behind a branch and the row's loads are all in
// flight together); the caller masks positions >= E.
template <int NC, class W>
PW_WAVE void load_row_scores(W &w, const float *scores_row, const float *bias, uint32_t E, float (&sc)[NC],
                             float (&b)[NC])
{
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t e = 64 * c + w.lane();
        const uint32_t ec = e < E ? e : E - 1;
        sc[c] = scores_row[ec];
        b[c] = bias[ec];
    }
}

// The largest value at positions [from, n) of the row (-inf when none).
template <int NC, class W>
PW_WAVE float wave_max_from(W &w, const WaveRow<NC> &a, uint32_t from, uint32_t n)
{
    float r = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t p = 64 * c + w.lane();
        if (p >= from && p < n)
            r = a.v[c] > r ? a.v[c] : r;
    }
    return w.max_all(r);
}

// One row of pytorch_noaux_routes (src/text_endpoint.rs:4394-4473) by one wave: corrected =
// score + bias for the row's E experts (E <= 64 NC), the top 8 in libc++ nth_element order, the
// boundary check against the best rejected value and the renormalised weights, with the arithmetic
// of noaux_finish_row8 spread over lanes 0..7 (lane k: route k, position k of the partitioned row):
// lanes (s0 + s4, s1 + s5, s2 + s6, s3 + s7) folded left to right from 0, + 1e-20, one division
// per lane, the weight sum folded in route order. Returns the row's RouteStatus on every lane; on
// ROUTE_OK lane k < 8 holds route k in sel_k / w_k and *tie is set.
template <int NC, class W>
PW_WAVE int select_route_row(W &w, const float *scores_row, const float *bias, uint32_t E, TopkEntry *lds,
                             uint32_t &sel_k, float &w_k, bool *tie)
{
    WaveRow<NC> a;
    uint32_t sb[NC];  // the uncorrected scores' bits, by position as loaded (= expert id)
    bool bad = false;
    float sc[NC], b[NC];
    load_row_scores<NC>(w, scores_row, bias, E, sc, b);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t e = 64 * c + w.lane();
        const bool in = e < E;
        bad |= in && (!finite_f32_bits(sc[c]) || !finite_f32_bits(b[c]));
        sb[c] = in ? f32_bits(sc[c]) : 0u;
        a.v[c] = in ? sc[c] + b[c] : -__builtin_inff();
        a.id[c] = in ? (int32_t)e : -1;
    }
    *tie = false;
    sel_k = 0u;
    w_k = 0.f;
    if (w.ballot(bad))
        return ROUTE_NONFINITE;
    w.mark();
    nth_element_wave_regs(w, a, 7u, E, lds);
    const float rejected = wave_max_from(w, a, 8u, E);
    // the uncorrected scores by expert id, through the LDS buffer (free after the partition)
    float *s_lds = (float *)lds;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t e = 64 * c + w.lane();
        if (e < E)
            s_lds[e] = f32_from(sb[c]);
    }
    w.lds_sync();
    const uint32_t lane = w.lane();
    const bool mine = lane < 8;
    const int32_t id = a.id[0];
    const float chosen = mine ? s_lds[id] : 0.f;
    // the eight ids are distinct (the row's positions hold a permutation of them); checked as the
    // reference checks its top-k result
    bool dup = false;
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
        const int32_t idj = w.readlane(id, j);  // every lane takes part in the lane read
        dup |= mine && lane != j && idj == id;
    }
    float bnd = mine ? a.v[0] : __builtin_inff();
#pragma unroll
    for (uint32_t off = 4; off > 0; off >>= 1) {
        const float o = w.shfl(bnd, lane ^ off);
        bnd = o < bnd ? o : bnd;
    }
    const float boundary = w.readlane(bnd, 0u);
    if (w.ballot(dup) || !finite_f32_bits(boundary) || boundary < rejected)
        return ROUTE_TOPK;
    *tie = boundary == rejected;
    const float pair = chosen + w.shfl(chosen, (lane + 4) & 63);
    float sum = 0.0f;
#pragma unroll
    for (uint32_t l = 0; l < 4; ++l)
        sum = sum + w.readlane(pair, l);
    const float denominator = sum + 1.0e-20f;
    const float wt = chosen / denominator;
    const bool badw = mine && (!finite_f32_bits(wt) || wt < 0.0f);
    float wsum = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k)
        wsum += w.readlane(wt, k);
    const float dev = wsum - 1.0f;
    if (w.ballot(badw) || (dev < 0.0f ? -dev : dev) > 1.0e-6f)
        return ROUTE_WEIGHTS;
    sel_k = (uint32_t)id;
    w_k = wt;
    return ROUTE_OK;
}

// The set of the eight experts select_route_row selects, without the partition, where the set does
// not depend on the partition order: every score and bias finite, every corrected score finite,
// and the eighth largest corrected score strictly above the ninth. nth_element then leaves exactly
// the eight largest corrected scores in positions 0..7 (equal values above the boundary are all
// among them, whatever their order), so picking the largest value, all of its copies at once,
// eight times at most, finds the same set. Writes the ids in ascending order to ids[0..7] and
// returns true; returns false (nothing written) otherwise: the caller runs select_route_row. The
// order of the eight ids, and so the weights' denominator, still needs the partition.
template <int NC, class W>
PW_WAVE bool fast_top8_set(W &w, const float *scores_row, const float *bias, uint32_t E, uint32_t *ids)
{
    float v[NC];
    bool bad = false;
    float sc[NC], b[NC];
    load_row_scores<NC>(w, scores_row, bias, E, sc, b);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t e = 64 * c + w.lane();
        const bool in = e < E;
        const float s = sc[c] + b[c];
        v[c] = in ? s : -__builtin_inff();
        bad |= in && (!finite_f32_bits(sc[c]) || !finite_f32_bits(b[c]) || !finite_f32_bits(s));
    }
    if (w.ballot(bad))
        return false;
    bool sel[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
        sel[c] = false;
    uint32_t picked = 0;  // wave-uniform
    for (int it = 0; it < 8 && picked < 8; ++it) {
        // the largest value not yet taken (positions past E hold -inf and are never taken: every
        // corrected score is finite and E > 8)
        float m = -__builtin_inff();
#pragma unroll
        for (int c = 0; c < NC; ++c)
            m = !sel[c] && v[c] > m ? v[c] : m;
        m = w.max_all(m);
        uint32_t cnt = 0;
        bool hit[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            hit[c] = !sel[c] && 64 * c + w.lane() < E && v[c] == m;
            cnt += popc64(w.ballot(hit[c]));
        }
        if (picked + cnt > 8)
            return false;  // copies of the eighth largest value also below the boundary: a tie
#pragma unroll
        for (int c = 0; c < NC; ++c)
            sel[c] = sel[c] || hit[c];
        picked += cnt;
    }
    uint32_t base = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint64_t m = w.ballot(sel[c]);
        if (sel[c])
            ids[base + w.below(m)] = 64 * c + w.lane();
        base += popc64(m);
    }
    return true;
}

}  // namespace pw
