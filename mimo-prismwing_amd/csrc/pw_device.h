// Device helpers for gfx950 (CDNA4): MFMA operand types, FP8 -> bf16 conversion, bf16 splitting,
// wave reductions, and the shared plan structures used by the kernels and the host runtime.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pw_numerics.h"

namespace pw {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;

// 16-byte global (not flat) load, so it is counted only by the vector-memory counter. Weights use
// it too: plain loads streamed 4-10% faster than nontemporal ones on gfx950 for every weight
// pattern here (16-row x 64-byte decode tiles, 96-row prefill tiles, dense GEMV rows), and the
// nontemporal form fetched ~7% more bytes from HBM.
__device__ __forceinline__ uint4 load_global16(const void *p)
{
    const u32x4 v = *(global_u32x4 *)p;
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Scalar-typed global load through a pointer that was itself read from memory (such pointers are
// generic, and would otherwise become flat loads that also wait on the LDS counter).
template <class T>
__device__ __forceinline__ T load_g(const T *p)
{
    return *(const __attribute__((address_space(1))) T *)p;
}

// Direct global -> LDS load of 16 bytes per lane (gfx950 global_load_lds_dwordx4): lane i's bytes
// land at lds_wave_base + 16 * i, where lds_wave_base is wave-uniform. The data never occupies
// VGPRs; completion is counted by the vector-memory counter, so the issuing wave must wait for
// vmcnt before a barrier that publishes the LDS rows to the other waves.
__device__ __forceinline__ void lds_load16(const void *src_lane, void *lds_wave_base)
{
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src_lane,
                                     (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

// Waits until at most N vector-memory operations of this wave are outstanding (gfx9 s_waitcnt
// encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt at their no-wait maxima). Loads
// complete in issue order, so this is "everything but the last N loads".
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt has six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier ordering LDS accesses only: outstanding global loads stay in flight across it,
// which __syncthreads() would wait for.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Error bits raised by kernels into the runtime's device error word. The low bits keep the
// meaning of the reference's Metal error word (kernels/block_fp8_gemv.metal, bits 1..128).
enum : uint32_t {
    FLAG_LANES = 1u,
    FLAG_QUANT_NONFINITE = 2u,
    FLAG_SWIGLU_NONFINITE = 4u,
    FLAG_REDUCE_NONFINITE = 16u,
    FLAG_ROUND_NONFINITE = 32u,
    FLAG_FUSED_SWIGLU_NONFINITE = 128u,
    FLAG_SCHEDULE = 256u,
    FLAG_OUTPUT_NONFINITE = 512u,
    FLAG_ROUTE = 1024u,
};

// A 16-row output tile of a projection: weight rows [w, w + 16*K), one scale row (all 16 rows sit
// in one 128-row scale block), output rows [out_row, out_row + valid).
struct ProjTile {
    const uint8_t *w;
    const float *s;
    uint32_t out_row;
    uint32_t valid;
};

// Per-expert device pointers of a routed-expert bank.
struct ExpertPtrs {
    const uint8_t *gate_w;
    const float *gate_s;
    const uint8_t *up_w;
    const float *up_s;
    const uint8_t *down_w;
    const float *down_s;
};
static_assert(sizeof(ExpertPtrs) == 48, "ExpertPtrs is copied as three 16-byte units");

// One routed expert's entry of the device schedule: its weights, its placement slots
// [off, off + cnt) and the token rows of its first 16 slots (read with the entry's scalar load,
// so the gate/up kernel can start its activation gather without a dependent load). Entries past
// the last routed expert have cnt = 0.
struct ActiveExpert {
    ExpertPtrs ep;
    uint32_t off;
    uint32_t cnt;
    uint16_t tok[16];
    uint32_t pad[2];
};
static_assert(sizeof(ActiveExpert) == 96, "ActiveExpert is read as 96 bytes");

// Entry a (wave-uniform) of a schedule table that an earlier launch wrote: read through the
// constant address space, so the whole entry comes in scalar loads in one round trip, and taken
// by an empty asm before the caller's early exits, so no part of it is fetched after them (a
// compiler that sinks the pointer loads below an exit adds a second dependent round trip).
__device__ __forceinline__ ActiveExpert load_entry(const ActiveExpert *table, uint32_t a)
{
    typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
    struct Raw {
        u32x8 q[3];
    };
    const __attribute__((address_space(4))) u32x8 *p = (const __attribute__((address_space(4))) u32x8 *)(table + a);
    Raw r;
    r.q[0] = p[0];
    r.q[1] = p[1];
    r.q[2] = p[2];
    asm volatile("" ::"s"(r.q[0]), "s"(r.q[1]), "s"(r.q[2]));
    return __builtin_bit_cast(ActiveExpert, r);
}

// Device-side routed schedule (ascending expert id, positions ascending per expert), the
// layout of the reference's BTreeMap<expert, [(position, weight)]> (src/text_endpoint.rs:4767-4775).
struct MoePlan {
    uint32_t n_active;        // U, distinct routed experts
    uint32_t n_placements;    // rows * top_k
    uint32_t max_count;       // largest placement count of any expert
    uint32_t rejected;        // routes rejected: placement tables left zero, the layer writes zeros
};

// MFMA wrappers (gfx950). 16x16 output tile, lane l holds D[4*(l/16)+i][l%16], i = 0..3.
__device__ __forceinline__ f32x4 mfma_bf16_16x16x32(bf16x8 a, bf16x8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// FP8 (OCP e4m3fn) x FP8, K = 128 per instruction, E8M0 scales fixed at 2^0.
__device__ __forceinline__ f32x4 mfma_fp8_16x16x128(i32x8 a, i32x8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// Eight e4m3fn bytes (two dwords) -> eight bf16 (exact: e4m3 values are bf16 values).
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi)
{
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    bf16x8 r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
}

// e4m3fn codes of two finite values in [-448, 448], round to nearest even, in the low 16 bits
// (a in the low byte): v_cvt_pk_fp8_f32, which on gfx950 writes OCP e4m3fn and gives the byte of
// encode_e4m3fn_rne for every f32 of that range (all 2,277,507,074 of them compared on MI355X,
// subnormals and both zeros included). Callers clamp and zero non-finite values first.
__device__ __forceinline__ uint32_t encode2_e4m3fn(float a, float b)
{
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// round_bf16 where a non-finite result is only flagged and never stored: the same bits for every
// finite input and for infinities; a NaN may come out as an infinity of its sign (still
// non-finite). Two instructions fewer than the select that keeps NaN payloads.
__device__ __forceinline__ float round_bf16_or_nonfinite(float v)
{
    const uint32_t b = f32_bits(v);
    return f32_from((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
}

// a / scale for the quantisers, from the correctly rounded reciprocal rcp = 1 / scale (one IEEE
// division per group instead of one per value): q = a * rcp, then Markstein's correction
// q + (a - q * scale) * rcp with the remainder exact by fused multiply-add (P. Markstein, IBM J.
// Res. Dev. 34(1), 1990), and the sign of q, which a zero remainder would otherwise drop from -0.
// Where the quotient is at least 2^-10 this equals a / scale bit for bit; below that it may differ
// by an ulp, and every value there encodes to an e4m3 zero of the same sign. Used only where a is
// a bf16 value and scale = max(m, 1e-10) / 448 for a bf16 group absmax m >= |a|: over that whole
// domain (every such (a, m) pair, 1,065,402,238 of them) the clamped e4m3 codes equal those of the
// IEEE quotient.
__device__ __forceinline__ float quant_ratio_bf16(float a, float scale, float rcp)
{
    const float q = a * rcp;
    return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q, scale, a), rcp, q), q);
}

__device__ __forceinline__ __bf16 bf16_from_bits(uint16_t u) { return __builtin_bit_cast(__bf16, u); }

// f32 -> three bf16 planes with x == hi + mid + lo exactly (normal range): each remainder is
// exact in f32 (the operands are within a factor of two) and the last one has at most 8
// significant bits. Mode A feeds all three planes to the bf16 MFMA so products stay exact and
// only the f32 accumulation order differs from the reference.
__device__ __forceinline__ uint16_t rne_bf16_bits(float v)
{
    const uint32_t b = f32_bits(v);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ void split3_bf16(float x, uint16_t &hi, uint16_t &mid, uint16_t &lo)
{
    hi = rne_bf16_bits(x);
    const float r1 = x - f32_from((uint32_t)hi << 16);
    mid = rne_bf16_bits(r1);
    const float r2 = r1 - f32_from((uint32_t)mid << 16);
    lo = rne_bf16_bits(r2);
}

// Eight bf16 from a 16-byte word (bf16 activations are used as they are).
__device__ __forceinline__ bf16x8 bf16x8_from_u4(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ bool finite_f32(float v) { return (f32_bits(v) & 0x7f800000u) != 0x7f800000u; }

// silu of a bf16 gate as the bf16-staged SwiGLU rounds it, round(g / (1 + e^-g))
// (bf16_staged_swiglu, kernels/block_fp8_gemv.metal:139-160; CPU src/text_endpoint.rs:5336-5343).
// One definition for every kernel that evaluates it (mode B decode gate/up, the prefill silu
// table, the elementwise staged SwiGLU), so the in-place and table forms give the same bits.
__device__ __forceinline__ float silu_bf16_staged(float g) { return round_bf16(g / (1.0f + expf(-g))); }

// One wave's primitives for code written against a wave policy (pw_select_wave.h): lane id,
// ballot, a lane's value (the lane index wave-uniform), the value of the lane below, the wave
// maximum, and LDS ordering between the wave's own lanes (its LDS operations complete in order).
struct DeviceWave {
    __device__ __forceinline__ uint32_t lane() const { return __lane_id(); }
    __device__ __forceinline__ uint64_t ballot(bool b) const { return __ballot(b); }
    __device__ __forceinline__ uint32_t readlane(uint32_t v, uint32_t l) const
    {
        return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
    }
    __device__ __forceinline__ int32_t readlane(int32_t v, uint32_t l) const
    {
        return __builtin_amdgcn_readlane(v, (int)l);
    }
    __device__ __forceinline__ float readlane(float v, uint32_t l) const
    {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)l));
    }
    __device__ __forceinline__ uint32_t below(uint64_t m) const
    {
        return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    }
    // v (wave-uniform) into lane l of a register
    __device__ __forceinline__ float writelane(float old, float v, uint32_t l) const { return lane() == l ? v : old; }
    __device__ __forceinline__ int32_t writelane(int32_t old, int32_t v, uint32_t l) const
    {
        return lane() == l ? v : old;
    }
    __device__ __forceinline__ float shift_up1(float v) const { return __shfl_up(v, 1, 64); }
    // the maximum of v over the wave (finite or infinite values; every lane active): within each
    // 16-lane row by DPP swaps (quads, half-row and row mirrors), then the four rows' maxima read
    // out as scalars
    template <int CTRL>
    __device__ __forceinline__ static float dpp(float v)
    {
        return __builtin_bit_cast(float,
                                  __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
    }
    __device__ __forceinline__ static float fmax2(float a, float b) { return b > a ? b : a; }
    __device__ __forceinline__ float max_all(float v) const
    {
        v = fmax2(v, dpp<0xb1>(v));   // quad_perm [1, 0, 3, 2]
        v = fmax2(v, dpp<0x4e>(v));   // quad_perm [2, 3, 0, 1]
        v = fmax2(v, dpp<0x141>(v));  // row_half_mirror
        v = fmax2(v, dpp<0x140>(v));  // row_mirror
        return fmax2(fmax2(readlane(v, 0u), readlane(v, 16u)), fmax2(readlane(v, 32u), readlane(v, 48u)));
    }
    __device__ __forceinline__ float shfl(float v, uint32_t src) const { return __shfl(v, (int)src, 64); }
    __device__ __forceinline__ void lds_sync() const { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
    __device__ __forceinline__ void mark() const {}
};

__device__ __forceinline__ void raise_flag(uint32_t *flags, uint32_t bit)
{
    if (flags)
        __hip_atomic_fetch_or(flags, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Eight consecutive activations (16 bytes of bf16 or 32 of f32) as f32.
template <typename T>
__device__ __forceinline__ void load_act8(const T *p, float (&v)[8]);
template <>
__device__ __forceinline__ void load_act8<float>(const float *p, float (&v)[8])
{
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <>
__device__ __forceinline__ void load_act8<uint16_t>(const uint16_t *p, float (&v)[8])
{
    const uint4 a = *(const uint4 *)p;
    const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = f32_from(u[i] << 16);
        v[2 * i + 1] = f32_from(u[i] & 0xffff0000u);
    }
}

// Maximum over the 16 lanes of a DPP row (lanes 16r .. 16r + 15 of a wave, all active): swaps
// within quads, then the half-row and row mirrors, each a v_max_f32 with a DPP operand (no LDS
// permute).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float m)
{
    m = fmaxf(m, dpp_f32<0xb1>(m));   // quad_perm [1, 0, 3, 2]
    m = fmaxf(m, dpp_f32<0x4e>(m));   // quad_perm [2, 3, 0, 1]
    m = fmaxf(m, dpp_f32<0x141>(m));  // row_half_mirror
    m = fmaxf(m, dpp_f32<0x140>(m));  // row_mirror
    return m;
}

// Dynamic FP8 quantisation of one 128-column activation group (dynamic_fp8_quantized_group128,
// kernels/block_fp8_gemv.metal:84-137; CPU dynamic_fp8_activations, src/text_endpoint.rs:3008-3051)
// by 16 lanes of one wave (lane16 = 0..15, eight consecutive values each): max |finite x| over
// the group, scale = max(m, 1e-10) / 448, codes = e4m3fn RNE of x / scale clamped to +-448,
// non-finite values quantised as 0 and flagged with FLAG_QUANT_NONFINITE.
template <typename T>
__device__ __forceinline__ void quant_group128_team(const T *__restrict__ x, uint32_t group, uint32_t lane16,
                                                    uint8_t *__restrict__ codes, float *__restrict__ scales,
                                                    uint32_t *flags)
{
    const size_t base = (size_t)group * 128 + lane16 * 8;
    float v[8];
    load_act8<T>(x + base, v);
    bool fin[8], all = true;
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        fin[i] = finite_f32(v[i]);
        all &= fin[i];
        m = fmaxf(m, fin[i] ? fabsf(v[i]) : 0.f);
    }
    if (!all)
        raise_flag(flags, FLAG_QUANT_NONFINITE);
    m = row16_max(m);  // maximum over the group's 16 lanes (one DPP row: callers run whole teams)
    // bf16 inputs: a bf16 maximum, so the scale needs no division (scale_of_bf16_max), one
    // division per group for the reciprocal and quant_ratio_bf16 per value (the same codes as
    // x / scale over every bf16 input); f32 inputs divide each value
    const float scale = sizeof(T) == 2 ? scale_of_bf16_max(m) : fmaxf(m, 1.0e-10f) / 448.0f;
    if (lane16 == 0)
        scales[group] = scale;
    const float rcp = 1.0f / scale;
    float n[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if constexpr (sizeof(T) == 2)
            n[i] = fin[i] ? quant_ratio_bf16(v[i], scale, rcp) : 0.f;
        else
            n[i] = fin[i] ? v[i] / scale : 0.f;
        n[i] = fminf(fmaxf(n[i], -448.f), 448.f);  // n is finite: the same as the clamp by comparisons
    }
    const uint32_t lo = encode2_e4m3fn(n[0], n[1]) | (encode2_e4m3fn(n[2], n[3]) << 16);
    const uint32_t hi = encode2_e4m3fn(n[4], n[5]) | (encode2_e4m3fn(n[6], n[7]) << 16);
    *(uint2 *)(codes + base) = make_uint2(lo, hi);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}

// Inclusive prefix sum over the wave (every lane active; lane l: v_0 + ... + v_l) by DPP moves:
// shifts by 1, 2, 4, 8 within each 16-lane row, then the totals of rows 0 and 2 (lanes 15 and 47)
// into rows 1 and 3 and the total of rows 0-1 (lane 31) into rows 2 and 3.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v)
{
    v += dpp_u32<0x111, 0xf>(v);  // row_shr:1
    v += dpp_u32<0x112, 0xf>(v);  // row_shr:2
    v += dpp_u32<0x114, 0xf>(v);  // row_shr:4
    v += dpp_u32<0x118, 0xf>(v);  // row_shr:8
    v += dpp_u32<0x142, 0xa>(v);  // row_bcast:15
    v += dpp_u32<0x143, 0xc>(v);  // row_bcast:31
    return v;
}

// The wave's maximum (every lane active), as a scalar: within each 16-lane row by DPP swaps, then
// the four rows' maxima.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, dpp_u32<0xb1, 0xf>(v));   // quad_perm [1, 0, 3, 2]
    v = max(v, dpp_u32<0x4e, 0xf>(v));   // quad_perm [2, 3, 0, 1]
    v = max(v, dpp_u32<0x141, 0xf>(v));  // row_half_mirror
    v = max(v, dpp_u32<0x140, 0xf>(v));  // row_mirror
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(r0, r1), max(r2, r3));
}

// Exclusive prefix sum over the workgroup (blockDim.x <= 1024, whole waves): DPP scans of each
// wave, then of the per-wave totals. `tmp` holds 33 words of LDS. Returns the total in *total.
__device__ inline uint32_t block_exclusive_scan(uint32_t v, uint32_t *tmp, uint32_t *total)
{
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    const uint32_t inc = wave_inclusive_scan(v);
    if (lane == 63)
        tmp[wave] = inc;
    __syncthreads();
    if (threadIdx.x < 64) {
        const uint32_t w = threadIdx.x < nw ? tmp[threadIdx.x] : 0u;
        const uint32_t wi = wave_inclusive_scan(w);
        if (threadIdx.x < nw)
            tmp[16 + threadIdx.x] = wi - w;  // exclusive wave offsets
        if (threadIdx.x == nw - 1)
            tmp[32] = wi;
    }
    __syncthreads();
    const uint32_t r = tmp[16 + wave] + inc - v;
    *total = tmp[32];
    __syncthreads();  // tmp is reused by the next scan
    return r;
}

}  // namespace pw
