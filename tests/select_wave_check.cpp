/* CPU check of the device router's register nth_element (pw_select_wave.h; test support, built by
 * tests/test_select_wave.py): the header's algorithm runs here with a 64-lane wave emulated by 64
 * threads (ballots, lane reads and the wave maximum exchange values through shared arrays between
 * barriers; a lane write of a wave-uniform value is each thread's own decision; LDS is plain memory
 * ordered by a barrier), and the whole row it leaves -- every
 * position, not only the first eight -- must equal the serial libc++ nth_element restatement of
 * pw_topk.h, which the reference's golden top-k orders pin. Rows: random, few-level ties, all
 * equal, ascending, descending, one high value, many equal maxima; lengths 9..1024; nth 7 (the
 * router) and other positions. Prints the number of rows and mismatches; exits 1 on a mismatch. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <barrier>
#include <random>
#include <thread>
#include <vector>

#include "pw_select_wave.h"

namespace {

struct Shared {
    std::barrier<> bar{64};
    bool b[64];
    uint32_t u[64];
    float f[64];
};

struct CpuWave {
    uint32_t lane_;
    Shared *sh;
    uint32_t lane() const { return lane_; }
    uint64_t ballot(bool v)
    {
        sh->b[lane_] = v;
        sh->bar.arrive_and_wait();
        uint64_t m = 0;
        for (int l = 0; l < 64; ++l)
            m |= (uint64_t)sh->b[l] << l;
        sh->bar.arrive_and_wait();
        return m;
    }
    uint32_t readlane(uint32_t v, uint32_t l)
    {
        sh->u[lane_] = v;
        sh->bar.arrive_and_wait();
        const uint32_t r = sh->u[l];
        sh->bar.arrive_and_wait();
        return r;
    }
    int32_t readlane(int32_t v, uint32_t l) { return (int32_t)readlane((uint32_t)v, l); }
    float readlane(float v, uint32_t l) { return pw::f32_from(readlane(pw::f32_bits(v), l)); }
    uint32_t below(uint64_t m) const { return (uint32_t)__builtin_popcountll(m & ((1ull << lane_) - 1)); }
    // the written value is wave-uniform, so every lane decides for itself
    float writelane(float old, float v, uint32_t l) const { return lane_ == l ? v : old; }
    int32_t writelane(int32_t old, int32_t v, uint32_t l) const { return lane_ == l ? v : old; }
    float shift_up1(float v)
    {
        sh->f[lane_] = v;
        sh->bar.arrive_and_wait();
        const float r = lane_ ? sh->f[lane_ - 1] : v;
        sh->bar.arrive_and_wait();
        return r;
    }
    float max_all(float v)
    {
        sh->f[lane_] = v;
        sh->bar.arrive_and_wait();
        float r = sh->f[0];
        for (int l = 1; l < 64; ++l)
            r = sh->f[l] > r ? sh->f[l] : r;
        sh->bar.arrive_and_wait();
        return r;
    }
    float shfl(float v, uint32_t src)
    {
        sh->f[lane_] = v;
        sh->bar.arrive_and_wait();
        const float r = sh->f[src & 63];
        sh->bar.arrive_and_wait();
        return r;
    }
    void lds_sync() { sh->bar.arrive_and_wait(); }
    void mark() const {}
};

template <int NC>
void run_wave(const std::vector<float> &vals, uint32_t nth, std::vector<pw::TopkEntry> &out, float *rejected)
{
    const uint32_t n = (uint32_t)vals.size();
    Shared sh;
    std::vector<pw::TopkEntry> lds(64 * NC);
    out.assign(n, pw::TopkEntry{0.f, -1});
    std::vector<std::thread> threads;
    for (uint32_t lane = 0; lane < 64; ++lane)
        threads.emplace_back([&, lane]() {
            CpuWave w{lane, &sh};
            pw::WaveRow<NC> a;
            for (int c = 0; c < NC; ++c) {
                const uint32_t p = 64 * c + lane;
                a.v[c] = p < n ? vals[p] : -__builtin_inff();
                a.id[c] = p < n ? (int32_t)p : -1;
            }
            pw::nth_element_wave_regs(w, a, nth, n, lds.data());
            const float rej = pw::wave_max_from(w, a, 8, n);
            for (int c = 0; c < NC; ++c) {
                const uint32_t p = 64 * c + lane;
                if (p < n)
                    out[p] = pw::TopkEntry{a.v[c], a.id[c]};
            }
            if (lane == 0)
                *rejected = rej;
        });
    for (auto &t : threads)
        t.join();
}

// select_route_row (the router's whole row: corrected scores, top 8, boundary, weights) on the
// emulated wave; status, ids, weight bits and tie into the outputs
template <int NC>
int route_wave(const std::vector<float> &scores, const std::vector<float> &bias, uint32_t sel[8], float wt[8],
               bool *tie)
{
    const uint32_t E = (uint32_t)scores.size();
    Shared sh;
    std::vector<pw::TopkEntry> lds(64 * NC);
    int status = -1;
    std::vector<std::thread> threads;
    for (uint32_t lane = 0; lane < 64; ++lane)
        threads.emplace_back([&, lane]() {
            CpuWave w{lane, &sh};
            uint32_t s_k;
            float w_k;
            bool t = false;
            const int st = pw::select_route_row<NC>(w, scores.data(), bias.data(), E, lds.data(), s_k, w_k, &t);
            if (lane < 8) {
                sel[lane] = s_k;
                wt[lane] = w_k;
            }
            if (lane == 0) {
                status = st;
                *tie = t;
            }
        });
    for (auto &t : threads)
        t.join();
    return status;
}

// fast_top8_set on the emulated wave: whether it decided the set, and the ids it wrote
template <int NC>
bool fast_wave(const std::vector<float> &scores, const std::vector<float> &bias, uint32_t ids[8])
{
    const uint32_t E = (uint32_t)scores.size();
    Shared sh;
    bool decided = false;
    std::vector<std::thread> threads;
    for (uint32_t lane = 0; lane < 64; ++lane)
        threads.emplace_back([&, lane]() {
            CpuWave w{lane, &sh};
            const bool d = pw::fast_top8_set<NC>(w, scores.data(), bias.data(), E, ids);
            if (lane == 0)
                decided = d;
        });
    for (auto &t : threads)
        t.join();
    return decided;
}

bool fast_any(const std::vector<float> &s, const std::vector<float> &b, uint32_t ids[8])
{
    const size_t n = s.size();
    if (n <= 64) return fast_wave<1>(s, b, ids);
    if (n <= 128) return fast_wave<2>(s, b, ids);
    if (n <= 256) return fast_wave<4>(s, b, ids);
    if (n <= 512) return fast_wave<8>(s, b, ids);
    return fast_wave<16>(s, b, ids);
}

int route_any(const std::vector<float> &s, const std::vector<float> &b, uint32_t sel[8], float wt[8], bool *tie)
{
    const size_t n = s.size();
    if (n <= 64) return route_wave<1>(s, b, sel, wt, tie);
    if (n <= 128) return route_wave<2>(s, b, sel, wt, tie);
    if (n <= 256) return route_wave<4>(s, b, sel, wt, tie);
    if (n <= 512) return route_wave<8>(s, b, sel, wt, tie);
    return route_wave<16>(s, b, sel, wt, tie);
}

void run_any(const std::vector<float> &vals, uint32_t nth, std::vector<pw::TopkEntry> &out, float *rej)
{
    const size_t n = vals.size();
    if (n <= 64) run_wave<1>(vals, nth, out, rej);
    else if (n <= 128) run_wave<2>(vals, nth, out, rej);
    else if (n <= 256) run_wave<4>(vals, nth, out, rej);
    else if (n <= 512) run_wave<8>(vals, nth, out, rej);
    else run_wave<16>(vals, nth, out, rej);
}

std::vector<float> pattern(int kind, uint32_t n, std::mt19937_64 &rng)
{
    std::vector<float> v(n);
    std::normal_distribution<float> normal(0.f, 1.f);
    std::uniform_int_distribution<int> level(0, 5), two(0, 1);
    for (uint32_t i = 0; i < n; ++i) {
        switch (kind) {
        case 0: v[i] = normal(rng); break;
        case 1: v[i] = (float)level(rng) * 0.25f; break;
        case 2: v[i] = 0.75f; break;
        case 3: v[i] = (float)i; break;
        case 4: v[i] = (float)(n - i); break;
        case 5: v[i] = i == n / 2 ? 3.f : -1.f; break;
        case 6: v[i] = two(rng) ? 1.f : normal(rng) - 4.f; break;   // many equal maxima
        default: v[i] = (float)(i % 7); break;                        // periodic
        }
    }
    return v;
}

}  // namespace

// argv[1]: rows per random pattern; argv[2] "quick": five lengths and two nth positions per row.
int main(int argc, char **argv)
{
    const int per = argc > 1 ? atoi(argv[1]) : 40;
    const bool quick = argc > 2 && strcmp(argv[2], "quick") == 0;
    std::mt19937_64 rng(20261202);
    const std::vector<uint32_t> lengths = quick ? std::vector<uint32_t>{9, 65, 256, 257, 1000}
                                                : std::vector<uint32_t>{9, 10, 17, 63, 64, 65, 100, 128, 200, 256,
                                                                        257, 300, 512, 1000, 1024};
    long rows = 0, mismatches = 0;
    for (uint32_t n : lengths)
        for (int kind = 0; kind < 8; ++kind)
            for (int t = 0; t < (kind == 0 || kind == 1 || kind == 6 ? per : 2); ++t) {
                const std::vector<float> vals = pattern(kind, n, rng);
                std::uniform_int_distribution<uint32_t> pick(0, n - 1);
                const uint32_t nths[] = {7u, t % 2 ? pick(rng) : n - 1, 0u};
                for (int r = 0; r < (quick ? 2 : 3); ++r) {
                    const uint32_t nth = nths[r];
                    std::vector<pw::TopkEntry> want(n), got;
                    for (uint32_t i = 0; i < n; ++i)
                        want[i] = pw::TopkEntry{vals[i], (int32_t)i};
                    pw::nth_element_libcxx(want.data(), want.data() + nth, want.data() + n);
                    float rej = 0.f;
                    run_any(vals, nth, got, &rej);
                    float want_rej = -__builtin_inff();
                    for (uint32_t i = 8; i < n; ++i)
                        want_rej = want[i].v > want_rej ? want[i].v : want_rej;
                    bool same = memcmp(&rej, &want_rej, 4) == 0;
                    for (uint32_t i = 0; i < n && same; ++i)
                        same = want[i].i == got[i].i && memcmp(&want[i].v, &got[i].v, 4) == 0;
                    ++rows;
                    if (!same) {
                        if (mismatches < 5)
                            printf("mismatch: n %u kind %d nth %u\n", n, kind, nth);
                        ++mismatches;
                    }
                }
            }
    // whole routed rows against the host routing (noaux_route_row): sigmoid-like scores with a
    // bias, tied scores, and a non-finite bias
    std::uniform_real_distribution<float> unit(0.f, 1.f), small(-0.01f, 0.01f);
    // trials 0..2 (and their repeats): random scores with a bias, five score levels with a bias, random
    // scores without one (trial 2: a NaN bias); then the rows the fast set must tell apart: five
    // levels without a bias (a tied boundary), a pair of equal values inside the top eight, the
    // top eight all equal with a lower ninth, and the eighth and ninth equal
    const int trials = quick ? 3 : 12;
    for (uint32_t E : {9u, 100u, 256u, 1000u})
        for (int t = 0; t < trials + 4; ++t) {
            std::vector<float> sc(E), bi(E);
            for (uint32_t e = 0; e < E; ++e) {
                sc[e] = t % 3 == 1 || t == trials ? (float)(e % 5) * 0.125f + 0.25f : unit(rng);
                bi[e] = t % 3 == 2 || t >= trials ? 0.f : small(rng);
            }
            if (t == 2)
                bi[E / 2] = __builtin_nanf("");
            if (t > trials) {
                std::vector<uint32_t> order(E);
                for (uint32_t e = 0; e < E; ++e)
                    order[e] = e;
                std::sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return sc[a] > sc[b]; });
                if (t == trials + 1)
                    sc[order[5]] = sc[order[2]];
                else if (t == trials + 2)
                    for (int k = 1; k < 8; ++k)
                        sc[order[k]] = sc[order[0]];
                else
                    sc[order[8]] = sc[order[7]];
            }
            uint32_t ws[8] = {}, hs[8] = {};
            float ww[8] = {}, hw[8] = {};
            bool wtie = false, htie = false;
            std::vector<pw::TopkEntry> scratch(E);
            const int want = pw::noaux_route_row(sc.data(), bi.data(), E, scratch.data(), hs, hw, &htie);
            const int got = route_any(sc, bi, ws, ww, &wtie);
            bool same = got == want;
            if (same && want == pw::ROUTE_OK) {
                same = wtie == htie;
                for (int k = 0; k < 8; ++k)
                    same = same && ws[k] == hs[k] && memcmp(&ww[k], &hw[k], 4) == 0;
            }
            ++rows;
            if (!same) {
                if (mismatches < 5)
                    printf("route mismatch: E %u trial %d status %d vs %d\n", E, t, got, want);
                ++mismatches;
            }
            // the fast set: decided exactly when every value is finite and the boundary is not tied
            // (a routed row: the host's status is ROUTE_OK), and then the host's eight ids
            uint32_t fids[8] = {};
            const bool decided = fast_any(sc, bi, fids);
            bool fsame = true;
            if (want == pw::ROUTE_OK) {
                fsame = decided == !htie;
                if (decided) {
                    uint32_t sorted[8];
                    memcpy(sorted, hs, sizeof sorted);
                    std::sort(sorted, sorted + 8);
                    fsame = fsame && memcmp(sorted, fids, sizeof sorted) == 0;
                }
            } else if (want == pw::ROUTE_NONFINITE) {
                fsame = !decided;
            }
            ++rows;
            if (!fsame) {
                if (mismatches < 5)
                    printf("fast set mismatch: E %u trial %d decided %d tie %d\n", E, t, decided, htie);
                ++mismatches;
            }
        }
    printf("rows %ld mismatches %ld\n", rows, mismatches);
    return mismatches != 0;
}
