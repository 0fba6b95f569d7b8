// The route weights of one batch row scheduled from its expert set alone (RouteJob): run by the
// standalone route_weights_kernel and by the extra workgroups of the decode layer's expert launches.
#pragma once

#include "pw_device.h"
#include "pw_launch.h"
#include "pw_select_wave.h"

namespace pw {

// Row p on one wave (lane = threadIdx.x & 63): select_route_row gives the routes in the
// reference's order, their renormalised weights and the tie flag; the routes are written out,
// checked to be the schedule's set, and each weight is written to its placement slot (the row's
// slots are in ascending expert id, so route k's slot is the row's slot of rank #{j: id_j < id_k}),
// or, with no schedule (row_slots null), to placement_w[8 p + i] for the set's i-th expert.
// A row whose routing fails (or whose set differs from the schedule's) gets ids E and zero
// weights, raises FLAG_ROUTE and FLAG_SCHEDULE and marks the batch rejected, as the schedule marks
// a batch with such routes: the combine then writes zeros. lds: 64 NC entries.
template <int NC>
__device__ __forceinline__ void route_weights_row(const RouteJob &j, uint32_t p, TopkEntry *lds)
{
    DeviceWave w;
    uint32_t sel_k;
    float w_k;
    bool tie = false;
    const int st = select_route_row<NC>(w, j.scores + (size_t)p * j.E, j.bias, j.E, lds, sel_k, w_k, &tie);
    const uint32_t lane = w.lane();
    const uint32_t prev = j.set_ids[(size_t)p * 8 + (lane & 7)];
    bool found = false;
    uint32_t rank = 0, pos = 0;
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t o = w.readlane(prev, k);  // every lane takes part in the lane reads
        found |= o == sel_k;
        pos = o == sel_k ? k : pos;
        rank += w.readlane(sel_k, k) < sel_k ? 1u : 0u;
    }
    const bool fail = st != ROUTE_OK || w.ballot(lane < 8 && !found) != 0;
    if (fail) {
        sel_k = j.E;
        w_k = 0.0f;
        tie = false;
    }
    if (lane < 8) {
        j.route_ids[(size_t)p * 8 + lane] = sel_k;
        j.route_w[(size_t)p * 8 + lane] = w_k;
        if (j.row_slots) {
            if (!fail && load_g(&j.plan->rejected) == 0u)
                j.placement_w[j.row_slots[(size_t)p * 8 + rank]] = w_k;
        } else {
            // no schedule: the weights in the set's order (a failed row: NaN weights, which the
            // one-token layer rejects as invalid routes)
            j.placement_w[(size_t)p * 8 + (fail ? lane : pos)] = fail ? __builtin_nanf("") : w_k;
        }
    }
    if (lane == 0) {
        if (fail) {
            j.plan->rejected = 1u;
            raise_flag(j.flags, FLAG_ROUTE | FLAG_SCHEDULE);
        }
        if (tie && j.tie_rows)
            atomicAdd(j.tie_rows, 1u);
    }
}

// The extra workgroups of an expert launch carrying a job (the first ROUTE_JOB_WGS of its grid):
// wave 0 of workgroup p < rows takes row p. Returns true for those workgroups, which then leave;
// the others see their own index less ROUTE_JOB_WGS in *bid.
__device__ __forceinline__ bool route_job_prologue(const RouteJob &j, void *lds, uint32_t *bid)
{
    *bid = blockIdx.x;
    if (j.rows == 0)
        return false;
    if (blockIdx.x >= ROUTE_JOB_WGS) {
        *bid = blockIdx.x - ROUTE_JOB_WGS;
        return false;
    }
    if (blockIdx.x < j.rows && threadIdx.x < 64)
        route_weights_row<4>(j, blockIdx.x, (TopkEntry *)lds);
    return true;
}

}  // namespace pw
