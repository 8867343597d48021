// px_scan_common.h -- device pieces shared by the MFMA scans of FlatIndex searches
// (px_flat.hip: per-split lists; px_collect.hip: threshold collect), gfx950, wave64.
#pragma once

#include "px_device.h"
#include "px_kernels.h"

namespace px {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4v __attribute__((ext_vector_type(4)));

constexpr int kTileRows = 64;            // corpus rows per tile: two 32-row MFMA blocks
constexpr int kChunk = 128;              // dims per staged K-chunk (16 groups of 8)
constexpr int kLdsStride = kChunk + 4;   // row pitch in LDS; +4 floats keeps b128 reads conflict-free

// v_mfma_f32_32x32x2f32 result layout: lane l, register r holds D[i][j] with
// j = l % 32 and i = 8 * (r / 4) + 4 * (l / 32) + r % 4.
__device__ __forceinline__ int mfma_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ f32x16 mfma4(float4 a, float4 b, f32x16 c) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, c, 0, 0, 0);
    return c;
}

// Stage sync of the collect scans (no barrier per stage): each wave publishes in an 8-word
// LDS array the last stage it has committed to a stage buffer (stage_publish, release), and
// waits with stage_wait until every wave has committed a given stage (acquire).
constexpr int kSpinLimit = 1 << 16;  // polls of a stage wait (each one s_sleep 1: ~5 ms)

// The launch's arguments with FlatScanArgs::spin_limit in force: kSpinLimit where it is 0.
inline FlatScanArgs with_spin_limit(const FlatScanArgs& a) {
    FlatScanArgs b = a;
    if (b.spin_limit <= 0) b.spin_limit = kSpinLimit;
    return b;
}

__device__ __forceinline__ void stage_publish(int* committed, int wave, int lane, int v) {
    if (lane == 0)
        __hip_atomic_store(committed + wave, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Polls until every word of the 8-word array is >= ct; addr: the LDS address of word
// lane & 7. Gives up after lim polls (lim >= 1; FlatScanArgs::spin_limit, normally
// kSpinLimit) and returns the number of polls: lim if it gave up (the caller reports it).
// One asm block: as a compiled loop in the middle of an unrolled stage it split the
// schedule and cost register spills. Its s_waitcnt makes the load acquire (LDS at workgroup
// scope needs no more), and the "memory" clobber keeps the stage buffer accesses after it.
// The poll count is early-clobber ("+&s"): as a plain in-out operand it may share a
// register with an equal input (it was given ct's, and each poll then raised the target).
__device__ __forceinline__ int stage_wait(unsigned addr, int ct, int lim) {
    int v, spins = 0;
    unsigned long long m;
    asm volatile(
        ".Lpx_poll%=:\n"
        "  ds_read_b32 %[v], %[addr]\n"
        "  s_waitcnt lgkmcnt(0)\n"
        "  v_cmp_lt_i32_e64 %[m], %[v], %[ct]\n"
        "  s_cmp_lg_u64 %[m], 0\n"
        "  s_cbranch_scc0 .Lpx_done%=\n"
        "  s_add_u32 %[sp], %[sp], 1\n"
        "  s_cmp_ge_u32 %[sp], %[lim]\n"
        "  s_cbranch_scc1 .Lpx_done%=\n"
        "  s_sleep 1\n"
        "  s_branch .Lpx_poll%=\n"
        ".Lpx_done%=:\n"
        : [v] "=&v"(v), [m] "=&s"(m), [sp] "+&s"(spins)
        : [addr] "v"(addr), [ct] "s"(ct), [lim] "s"(lim)
        : "memory", "scc");
    return spins;
}

// Of a SIMD's pair of waves (w and w ^ 4), the one behind issues first: the matrix unit
// otherwise favours the older wave, which runs the one stage ahead the stage buffers allow
// and then idles at its wait while the other finishes and commits. partner_committed: the
// partner's published stage; mine: this wave's (the partner is behind when it is not past).
__device__ __forceinline__ void pair_priority(int partner_committed, int mine) {
    if (partner_committed > mine) __builtin_amdgcn_s_setprio(2);
    else __builtin_amdgcn_s_setprio(0);
}

// Total-order int of a key (flat.rs:30's f32::total_cmp) and back; the mapping is its own
// inverse. Shared thresholds are published as these ints with atomicMin.
__device__ __forceinline__ float from_total_key(int t) {
    return __int_as_float(t ^ (int)(((unsigned)(t >> 31)) >> 1));
}

// fp32 MFMA tiles starting from zero accumulators.
__device__ __forceinline__ f32x16 mfma4z(float4 a, float4 b) {
    const f32x16 z = {0.f};
    f32x16 c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, z, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, c, 0, 0, 0);
    return c;
}

// fp16 operands, fp32 accumulation: v_mfma_f32_32x32x16_f16 (gfx950), 16 dims a tile. Lane l
// holds row l % 32 (A) or column l % 32 (B) at dims 8 (l / 32) .. 8 (l / 32) + 7; the
// result layout is the fp32 tiles' (mfma_row). Products of fp16 values are exact in fp32.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x16 mfma16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma16z(f16x8 a, f16x8 b) {
    const f32x16 z = {0.f};
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, z, 0, 0, 0);
}
// One dim group of a 128-dim chunk: 8 dims (fp32, four tiles) or 16 (fp16, one tile).
__device__ __forceinline__ f32x16 mfma_group(float4 a, float4 b, f32x16 c) { return mfma4(a, b, c); }
__device__ __forceinline__ f32x16 mfma_group(f16x8 a, f16x8 b, f32x16 c) { return mfma16(a, b, c); }
__device__ __forceinline__ f32x16 mfma_group_z(float4 a, float4 b) { return mfma4z(a, b); }
__device__ __forceinline__ f32x16 mfma_group_z(f16x8 a, f16x8 b) { return mfma16z(a, b); }

// Slots h * 16 .. h * 16 + 15 of a query's shared-bound slots (FlatScanArgs::gbest,
// slot-major: q_slots = gbest + q, slot s at q_slots[s * ld]), relaxed device-scope loads
// (other workgroups publish them with atomicMin). The addresses are stepped from a pointer
// the empty asm makes opaque here: sixteen per-lane 64-bit offsets formed from h and ld
// alone were hoisted out of the callers' scan loops and spilled.
__device__ __forceinline__ void load_slots16(const int* q_slots, int64_t ld, int h,
                                             int (&v)[16]) {
    const int* p = q_slots;
    asm volatile("" : "+v"(p));
    p += (int64_t)h * 16 * ld;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        v[u] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        p += ld;
    }
}

// rank-th smallest (1-based, rank <= 32) of the 32 ints held as v[0..15] by this lane and
// by lane ^ 32; both lanes return it. Bitonic: sort 16 in registers, split the union into
// its 16 smallest and 16 largest with the partner's list reversed, sort those halves.
__device__ __forceinline__ int kth_smallest32(int (&v)[16], int rank) {
#pragma unroll
    for (int k = 2; k <= 16; k <<= 1)
#pragma unroll
        for (int s = k >> 1; s > 0; s >>= 1)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int l = i ^ s;
                if (l > i) {
                    const int mn = min(v[i], v[l]), mx = max(v[i], v[l]);
                    const bool up = (i & k) == 0;
                    v[i] = up ? mn : mx;
                    v[l] = up ? mx : mn;
                }
            }
    // only the half holding the answer is kept (rank is uniform across the wave)
    const bool low = rank <= 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int p = __shfl_xor(v[15 - i], 32);
        v[i] = low ? min(v[i], p) : max(v[i], p);
    }
#pragma unroll
    for (int s = 8; s > 0; s >>= 1)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int l = i ^ s;
            if (l > i) {
                const int mn = min(v[i], v[l]), mx = max(v[i], v[l]);
                v[i] = mn;
                v[l] = mx;
            }
        }
    const int want = low ? rank - 1 : rank - 17;
    int r = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 16; ++i) r = i == want ? v[i] : r;
    return r;
}

// kl-th smallest (kl <= 64) key of the 64 rows a lane pair holds for query j in the first
// tile of a split (key[x] is row 32 (x / 16) + mfma_row(x % 16, h)); rows at or past rem,
// and padding queries, do not count. +inf when fewer than kl rows count. kl rounds of
// "smallest remaining" over the pair, as in first_tile_lists, keeping only the value.
__device__ __forceinline__ float first_tile_kth(const float (&key)[32], int rem, bool qvalid,
                                                int kl) {
    constexpr int kNoKey = 0x7fffffff;
    const int h = lane_id() >> 5;
    int tk[32];
#pragma unroll
    for (int x = 0; x < 32; ++x) {
        const int off = (x >> 4) * 32 + mfma_row(x & 15, h);
        tk[x] = (qvalid && off < rem) ? total_key(key[x]) : kNoKey;
    }
    int last = kNoKey;
    for (int r = 0; r < kl; ++r) {
        int bt = kNoKey, bx = 0;
#pragma unroll
        for (int x = 0; x < 32; ++x) {
            const bool lt = tk[x] < bt;
            bt = lt ? tk[x] : bt;
            bx = lt ? x : bx;
        }
        const int pt = __shfl_xor(bt, 32);
        // equal minima: the h == 0 lane's goes first (the partner agrees)
        const bool mine = bt < pt || (bt == pt && h == 0);
        last = mine ? bt : pt;
        if (__ballot(last != kNoKey) == 0) break;  // no query has a row left
#pragma unroll
        for (int x = 0; x < 32; ++x) tk[x] = (mine && x == bx) ? kNoKey : tk[x];
    }
    return last == kNoKey ? __int_as_float(0x7f800000) : from_total_key(last);
}

}  // namespace px
