// px_device.h -- device-side helpers shared by the flat and PQ kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace px {

// Index checks of the debug build (-DPX_DEBUG, libproxima_px_debug.so). A failed check does
// not trap: the first failure's file and line (file_id * 100000 + line) are recorded in the
// launch's debug word (dbg, one device int the host clears before a search and reads after
// it), and the search fails with PX_ERR_ARG naming them. In the product build the checks
// compile to nothing.
#ifdef PX_DEBUG
#define PX_DCHECK(dbg, file_id, cond)                                          \
    do {                                                                       \
        if ((dbg) != nullptr && !(cond)) atomicCAS((dbg), 0, (file_id) * 100000 + __LINE__); \
    } while (0)
#else
#define PX_DCHECK(dbg, file_id, cond) \
    do {                              \
    } while (0)
#endif
constexpr int kDbgFlat = 1, kDbgCollect = 2, kDbgPq = 3;

// Id sentinel for an empty list slot. Real ids (row numbers or compacted positions)
// are < 2^31 - 1, so the sentinel sorts after every real candidate of equal key.
constexpr int kIdNone = 0x7fffffff;

// The IEEE-754 totalOrder mapping used by f32::total_cmp (crates/core/src/flat.rs:20):
// negative numbers get their magnitude bits flipped, then keys compare as int32.
__device__ __forceinline__ int total_key(float f) {
    int b = __float_as_int(f);
    return b ^ (int)(((unsigned)(b >> 31)) >> 1);
}

// The largest float below v (v not NaN; -inf stays -inf), so that for every non-NaN key,
// key <= next_below(v) is exactly key < v (with -0 == +0 as float compares have them).
__device__ __forceinline__ float next_below(float v) {
    const int b = __float_as_int(v);
    if (v > 0.f) return __int_as_float(b - 1);
    if (v == 0.f) return __int_as_float((int)0x80000001);
    return v == -__int_as_float(0x7f800000) ? v : __int_as_float(b + 1);
}

// Canonical candidate order: (key in total order, id) lexicographic.
__device__ __forceinline__ bool cand_less(float ka, int ia, float kb, int ib) {
    int ta = total_key(ka), tb = total_key(kb);
    return ta < tb || (ta == tb && ia < ib);
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int readlane_i(int v, int lane) {
    return __builtin_amdgcn_readlane(v, lane);
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }

// List slot ids: int positions, or (to fit the lists of eight waves beside three stage
// buffers, or more waves beside two) 16-bit offsets from the split's first position with
// 0xffff as the empty sentinel.
template <typename IdT>
__device__ __forceinline__ int id_load(IdT v, int base) {
    if constexpr (sizeof(IdT) == 2) return v == 0xffff ? kIdNone : base + (int)v;
    else return (int)v;
}
template <typename IdT>
__device__ __forceinline__ IdT id_store(int id, int base) {
    if constexpr (sizeof(IdT) == 2) return (IdT)(id == kIdNone ? 0xffff : id - base);
    else return (IdT)id;
}

// Wave-cooperative insertion of (ck, cid) into a sorted list of `kl` live slots
// (capacity KP) held in LDS at lk/li. Lane s owns slots s, s+64, ... The caller guarantees
// (ck, cid) is smaller than slot kl-1, so the new element lands at some pos < kl and the
// old slot kl-1 falls off the end. Returns the new last live slot (the list threshold) in
// every lane.
template <int KP, typename IdT>
__device__ __forceinline__ void list_insert(float* lk, IdT* li, int base, int kl, float ck,
                                            int cid, float& tau_k, int& tau_i) {
    const int s = lane_id();
    constexpr int U = (KP + 63) / 64;
    float okey[U], pkey[U];
    int oid[U], pid[U];
    unsigned long long after[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int slot = s + 64 * u;
        const bool live = slot < kl;
        okey[u] = live ? lk[slot] : __int_as_float(0x7f800000);
        oid[u] = live ? id_load(li[slot], base) : kIdNone;
        if constexpr (U == 1) {
            // slot s - 1 is lane s - 1's okey: a DPP wave_shr:1 (lane 0 keeps 0; it never
            // shifts) rather than two more LDS reads on the insertion's critical path
            pkey[u] = __int_as_float(
                __builtin_amdgcn_update_dpp(0, __float_as_int(okey[u]), 0x138, 0xF, 0xF, false));
            pid[u] = __builtin_amdgcn_update_dpp(0, oid[u], 0x138, 0xF, 0xF, false);
        } else {
            pkey[u] = (live && slot > 0) ? lk[slot - 1] : 0.f;
            pid[u] = (live && slot > 0) ? id_load(li[slot - 1], base) : 0;
        }
        after[u] = __ballot(live && cand_less(ck, cid, okey[u], oid[u]));
    }
    int pos = kl;
#pragma unroll
    for (int u = U - 1; u >= 0; --u)
        if (after[u]) pos = 64 * u + __builtin_ctzll(after[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int slot = s + 64 * u;
        if (slot < kl) {
            if (slot > pos) {
                lk[slot] = pkey[u];
                li[slot] = id_store<IdT>(pid[u], base);
            } else if (slot == pos) {
                lk[slot] = ck;
                li[slot] = id_store<IdT>(cid, base);
            }
        }
    }
    // new threshold: slot kl-1 after the shift
    const int last = kl - 1;
    float nk;
    int ni;
    if (pos == last) {
        nk = ck;
        ni = cid;
    } else {
        // slot kl-1 now holds what was in slot kl-2, i.e. pkey of the lane owning kl-1
        const int owner = last & 63, uu = last >> 6;
        float pk = pkey[0];
        int pi = pid[0];
#pragma unroll
        for (int u = 1; u < U; ++u)
            if (uu == u) { pk = pkey[u]; pi = pid[u]; }
        nk = readlane_f(pk, owner);
        ni = readlane_i(pi, owner);
    }
    tau_k = nk;
    tau_i = ni;
}

// ---------------------------------------------------------------------------
// The reference's arithmetic (crates/core/src/distance.rs:3-39): eight lane
// accumulators over chunks of 8, lane sum in order, then the remainder, no FMA.
// Every translation unit is built with -ffp-contract=off; FMAs elsewhere are explicit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float ref_l2_sqr(const float* a, const float* b, int n) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int chunks = n >> 3;
    for (int c = 0; c < chunks; ++c) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float d = a[c * 8 + l] - b[c * 8 + l];
            acc[l] = acc[l] + d * d;
        }
    }
    float sum = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) sum = sum + acc[l];
    for (int i = chunks * 8; i < n; ++i) {
        const float d = a[i] - b[i];
        sum = sum + d * d;
    }
    return sum;
}

__device__ __forceinline__ float ref_inner_product(const float* a, const float* b, int n) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int chunks = n >> 3;
    for (int c = 0; c < chunks; ++c) {
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[l] = acc[l] + a[c * 8 + l] * b[c * 8 + l];
    }
    float sum = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) sum = sum + acc[l];
    for (int i = chunks * 8; i < n; ++i) sum = sum + a[i] * b[i];
    return sum;
}

// Same arithmetic and order, spread over a group of 8 consecutive lanes (gl = lane % 8, all
// 8 lanes of the group active and on the same a, b): lane gl accumulates the reference's
// accumulator gl over the chunks in order -- each of its loads independent of the others,
// so one round trip to memory instead of one per 4 chunks -- then every lane of the group
// folds the 8 accumulators from 0.0 in order and adds the remainder, as ref_l2_sqr /
// ref_inner_product do. Pitches a multiple of 8 floats.
__device__ __forceinline__ float ref_key_g8(const float* a, const float* b, int n, bool l2,
                                           int gl) {
    float acc = 0.f;
    const int chunks = n >> 3;
#pragma unroll 8
    for (int c = 0; c < chunks; ++c) {
        const float x = a[c * 8 + gl], y = b[c * 8 + gl];
        if (l2) {
            const float d = x - y;
            acc = acc + d * d;
        } else {
            acc = acc + x * y;
        }
    }
    const int base = (int)(threadIdx.x & 63) & ~7;
    float sum = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) sum = sum + __shfl(acc, base + l, 64);
    for (int i = chunks * 8; i < n; ++i) {
        if (l2) {
            const float d = a[i] - b[i];
            sum = sum + d * d;
        } else {
            sum = sum + a[i] * b[i];
        }
    }
    return sum;
}

// Same arithmetic and order, for rows stored with a pitch that is a multiple of 8 floats
// (32-byte aligned, readable up to the next multiple of 8): chunks of 8 are loaded as two
// float4, four chunks per step so that the loads of a step are in flight together.
__device__ __forceinline__ float ref_key_v(const float* a, const float* b, int n, bool l2) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int chunks = n >> 3;
    auto step = [&](const float4 (&x)[2], const float4 (&y)[2]) {
        const float xs[8] = {x[0].x, x[0].y, x[0].z, x[0].w, x[1].x, x[1].y, x[1].z, x[1].w};
        const float ys[8] = {y[0].x, y[0].y, y[0].z, y[0].w, y[1].x, y[1].y, y[1].z, y[1].w};
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            if (l2) {
                const float d = xs[l] - ys[l];
                acc[l] = acc[l] + d * d;
            } else {
                acc[l] = acc[l] + xs[l] * ys[l];
            }
        }
    };
    int c = 0;
    for (; c + 4 <= chunks; c += 4) {
        float4 x[4][2], y[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            x[u][0] = *reinterpret_cast<const float4*>(a + (c + u) * 8);
            x[u][1] = *reinterpret_cast<const float4*>(a + (c + u) * 8 + 4);
            y[u][0] = *reinterpret_cast<const float4*>(b + (c + u) * 8);
            y[u][1] = *reinterpret_cast<const float4*>(b + (c + u) * 8 + 4);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) step(x[u], y[u]);
    }
    for (; c < chunks; ++c) {
        float4 x[2], y[2];
        x[0] = *reinterpret_cast<const float4*>(a + c * 8);
        x[1] = *reinterpret_cast<const float4*>(a + c * 8 + 4);
        y[0] = *reinterpret_cast<const float4*>(b + c * 8);
        y[1] = *reinterpret_cast<const float4*>(b + c * 8 + 4);
        step(x, y);
    }
    float sum = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) sum = sum + acc[l];
    for (int i = chunks * 8; i < n; ++i) {
        if (l2) {
            const float d = a[i] - b[i];
            sum = sum + d * d;
        } else {
            sum = sum + a[i] * b[i];
        }
    }
    return sum;
}

}  // namespace px
