// px_collect16.hip -- the fp16 collect scan of FlatIndex searches for gfx950, 64 queries a
// wave.
//
// Replaces the per-query full scan of crates/core/src/flat.rs:106-148 on the collect path
// where the rows and the queries are exact in fp16 (FlatScanArgs::corpus_h / queries_h, rows
// of one 128-dim chunk): every row whose key (||x||^2 - 2 q.x for L2, -q.x for IP) is at or
// below its query's threshold, and at or below the splits' shared bound (DYN), is appended to
// a candidate region; flat_collect_select_kernel re-ranks the best k + 8 in the reference's
// arithmetic (distance.rs:3-39). Each product of fp16 values is exact, so the keys are the
// fp32 scan's up to the rounding of the sums, and the re-rank makes the results identical.
//
// Shape. One workgroup = 8 waves = 512 query slots x one corpus split. A wave holds 64
// queries as two 32-query B operands of v_mfma_f32_32x32x16_f16 (8 dim groups of 16 a query
// block: 64 VGPRs) and multiplies 32-row tiles: a tile's A operand for a dim group (one
// 16-byte LDS read a lane) feeds both query blocks' MFMAs. With 32 queries a wave on 64-row
// tiles (flat_collect_kernel's shape) each A read fed one MFMA, and the A reads of a tile
// took the LDS as many cycles as the tile's MFMAs took the matrix units; here they take half,
// and the corpus staged through LDS per query is halved too.
//
// Keys from the matrix unit. A tile's accumulators start from -||x||^2 / 2 of its rows (L2;
// zero for IP), so the MFMAs leave D = q.x - ||x||^2 / 2 = key / f with f = -2 (L2) or D =
// q.x = key / f with f = -1 (IP); every scaling is by a power of two, exact. The key tests
// compare D with ctest / f (at or above it: f is negative) and only an appended row's key is
// formed (f D), so no vector instruction a key is spent turning dot products into keys (on
// integer data below 2^23 the sums, and so the keys, are exact as before).
//
// Pipeline (as flat_collect_kernel's): three LDS stage buffers of 128 rows (4 tiles); the
// global loads of stage s + 2 are held in registers during stage s and written to its buffer
// at the end of stage s, after a barrier-free stage sync (every wave has committed stage
// s + 1: stage_wait). Two accumulator sets alternate between tiles: while tile t's MFMAs
// accumulate into one, the keys of tile t - 1 are formed in place from the other and
// pre-screened four to a dim group between the MFMAs. Row norms (L2) sit in sixteen 32-row
// slots, one a tile.
//
// Regions. Lane (j, h) of wave w holds query slots 64 w + j (block 0) and 64 w + 32 + j
// (block 1) of the workgroup's 512, and rows mfma_row(x, h) (x < 16) of each tile; so each
// slot has two regions per split, one per lane of its pair, in flat_collect_kernel's layout
// ([slot][split][h][cap]), and the select is shared.
#include "px_device.h"
#include "px_kernels.h"
#include "px_scan_common.h"

#include <float.h>

#include <type_traits>

namespace px {

namespace {

constexpr int kWaves16 = 8;
constexpr int kQueriesPerBlock16 = 64 * kWaves16;  // 512 query slots a workgroup
constexpr int kTile16 = 32;                        // rows a tile: one MFMA block
constexpr int kTilesPerStage16 = 4;
constexpr int kStage16 = kTile16 * kTilesPerStage16;  // 128 rows a stage
constexpr int kRowBytes16 = kChunk * 2;               // a staged fp16 row: 256 bytes
// LDS row pitch: 16 bytes more, so that sixteen consecutive rows' same 16-byte piece fall in
// sixteen different bank groups (conflict-free b128 reads of the A operands)
constexpr int kPitch16 = kRowBytes16 + 16;
constexpr int kBufs16 = 3;       // LDS stage buffers
constexpr int kNormSlots16 = 16;  // norm slots, one a tile (tiles t - 1 .. t + 11 in use)

// kl-th smallest (kl <= 32) key of the 32 rows a lane pair holds for one query block of a
// split's first tile (keys f acc[x], row mfma_row(x, h)); rows at or past rem, and padding
// queries, do not count; +inf when fewer than kl rows count. kl rounds of "smallest
// remaining" over the pair, as first_tile_kth does for 64-row tiles.
__device__ __forceinline__ float first_tile_kth16(const f32x16& acc, float f, int rem,
                                                  bool qvalid, int kl) {
    constexpr int kNoKey = 0x7fffffff;
    const int h = lane_id() >> 5;
    int tk[16];
#pragma unroll
    for (int x = 0; x < 16; ++x)
        tk[x] = (qvalid && mfma_row(x, h) < rem) ? total_key(f * acc[x]) : kNoKey;
    int last = kNoKey;
    for (int r = 0; r < kl; ++r) {
        int bt = kNoKey, bx = 0;
#pragma unroll
        for (int x = 0; x < 16; ++x) {
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
        for (int x = 0; x < 16; ++x) tk[x] = (mine && x == bx) ? kNoKey : tk[x];
    }
    return last == kNoKey ? __int_as_float(0x7f800000) : from_total_key(last);
}

// Largest of three / two D values as one v_max3_f32 / v_max_f32: fmaxf of values the compiler
// cannot prove canonical (MFMA results) costs two canonicalising instructions more (IEEE
// maxNum); D values are finite here (every row and query finite, checked on entry). The
// operands are MFMA results of the previous tile, far past any MFMA-to-VALU hazard window.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float max_raw(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

template <bool L2, bool FILT, bool DYN>
__global__ __launch_bounds__(512) void flat_collect16_kernel(FlatScanArgs a) {
    constexpr int NT = 512;
    constexpr int kF4PerRow = kRowBytes16 / 16;  // 16-byte pieces a staged row (16)
    constexpr int kRowStep = NT / kF4PerRow;     // rows between a thread's loads (32)
    constexpr int kPF = kStage16 / kRowStep;     // pieces a thread a stage (4)
    constexpr int NG = kChunk / 16;              // dim groups (8)
    constexpr float kF = L2 ? -2.0f : -1.0f;     // key = kF * D (below)
    static_assert(kPF == 4 && NG == 8, "four staged pieces a thread, eight dim groups");
    __shared__ __attribute__((aligned(16))) char tile[kBufs16][kStage16 * kPitch16];
    __shared__ __attribute__((aligned(16))) float tnorm[kNormSlots16][kTile16];
    // per wave: the last stage it has committed to a stage buffer (the stage sync below)
    __shared__ int committed[8];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    // query tiles in reverse launch order: the last (partial) tile, whose workgroups run
    // fastest, starts in the first round of workgroups with all its splits together
    const int qtiles = gridDim.x / a.splits;
    const int qt = qtiles - 1 - (int)(blockIdx.x / a.splits), split = blockIdx.x % a.splits;
    const int slot0 = qt * kQueriesPerBlock16 + wave * 64 + j;  // block 1: slot0 + 32
    // positions, tiles and stages fit 32 bits (at most 2^31 - 2 rows; host-checked)
    const int row0 = (int)((int64_t)split * a.rows_per_split);
    const int row1 = (int)min(a.n_eff, (int64_t)row0 + a.rows_per_split);
    PX_DCHECK(a.dbg, kDbgCollect, row0 < row1 && (int64_t)qtiles * a.splits == (int64_t)gridDim.x);
    const float kInf = __int_as_float(0x7f800000);
    const int ntiles = (row1 - row0 + kTile16 - 1) / kTile16;  // >= 1
    const int nstages = (ntiles + kTilesPerStage16 - 1) / kTilesPerStage16;
    const int cc = tid % kF4PerRow;   // this thread's 16-byte piece of a staged row
    const int rr0 = tid / kF4PerRow;  // its first row of a stage

    // ---- staging: row ids, global loads held in registers, commit to LDS ----------------
    // Every load is unconditional with a clamped address (rows past the split's end read
    // row 0): such rows' keys are never tested.
    // Addresses used now and then are formed where they are used, from an int the empty asm
    // makes opaque there: the compiler otherwise hoists them out of the scan loop as 64-bit
    // registers, which spill, and each stage end's reload then waited for every store in
    // flight.
    auto opaque = [](int v) __attribute__((always_inline)) {
        asm volatile("" : "+v"(v));
        return v;
    };
    int rid[kPF], pid;
    auto stage_ids = [&](int st) __attribute__((always_inline)) {
        // (positions past the split's end are formed in 64 bits: near 2^31 rows they overflow)
        const int64_t t0 = (int64_t)row0 + (int64_t)st * kStage16;
#pragma unroll
        for (int u = 0; u < kPF; ++u) {
            const int64_t pos = t0 + rr0 + u * kRowStep;
            const int v = FILT ? a.rowidx[min(pos, (int64_t)row1 - 1)] : (int)pos;
            rid[u] = pos < row1 ? v : -1;
            PX_DCHECK(a.dbg, kDbgCollect, pos >= row1 || (v >= 0 && v < a.rows));
        }
        const int64_t pos = t0 + tid;
        const int v = FILT ? a.rowidx[min(pos, (int64_t)row1 - 1)] : (int)pos;
        pid = (tid < kStage16 && pos < row1) ? v : -1;
    };
    float4 pf0, pf1, pf2, pf3;  // separate variables: an array of them ended up in memory
    float pn = 0.f;
    auto fetch = [&]() __attribute__((always_inline)) {
        const unsigned short* base = a.corpus_h + cc * 8;
        pf0 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[0], 0) * kChunk);
        pf1 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[1], 0) * kChunk);
        pf2 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[2], 0) * kChunk);
        pf3 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[3], 0) * kChunk);
        if (L2) pn = a.norms[max(pid, 0)];
    };
    auto commit = [&](int st, int buf) __attribute__((always_inline)) {
        char* tb = tile[buf] + rr0 * kPitch16 + cc * 16;
        *reinterpret_cast<float4*>(tb) = pf0;
        *reinterpret_cast<float4*>(tb + kRowStep * kPitch16) = pf1;
        *reinterpret_cast<float4*>(tb + 2 * kRowStep * kPitch16) = pf2;
        *reinterpret_cast<float4*>(tb + 3 * kRowStep * kPitch16) = pf3;
        // the stage's four tiles' accumulator starts -||x||^2 / 2, one slot a tile
        if (L2 && tid < kStage16)
            tnorm[(kTilesPerStage16 * st + (tid >> 5)) & (kNormSlots16 - 1)][tid & 31] =
                -0.5f * pn;
    };

    // prologue: stages 0 and 1 in LDS, ids of stage 2
    stage_ids(0);
    fetch();
    commit(0, 0);
    stage_ids(1);
    fetch();
    commit(1, 1);
    stage_ids(2);
    if (tid < 8) committed[tid] = 1;
    __syncthreads();

    // Stage sync without a barrier per stage (flat_collect_kernel's): each wave publishes
    // the last stage it has committed, and at the end of stage s waits until every wave has
    // committed stage s + 1 before it reads stage s + 1's buffer and writes stage s + 2's
    // (which held stage s - 1: a wave commits s + 1 only after all its reads of s - 1). A
    // wait gives up after a.spin_limit polls and reports it (a.spin_fail).
    const unsigned caddr = (unsigned)(uintptr_t)(committed + (lane & 7));
    auto wait_committed = [&](int ct) __attribute__((always_inline)) {
        if (stage_wait(caddr, ct, a.spin_limit) >= a.spin_limit && a.spin_fail && lane == 0)
            atomicOr(a.spin_fail, 1);
    };

    // A wave whose 64 query slots are all padding only helps stage the corpus: same loads,
    // same waits.
    if (qt * kQueriesPerBlock16 + wave * 64 >= a.nq) {
        int wb = 2;
        for (int s = 0; s < nstages; ++s) {
            fetch();
            stage_ids(s + 3);
            wait_committed(s + 1);
            commit(s + 2, wb);
            stage_publish(committed, wave, lane, s + 2);
            wb = wb == kBufs16 - 1 ? 0 : wb + 1;
        }
        return;
    }

    // ---- per-query state, [query block] --------------------------------------------------
    bool qvalid[2];
    int qidx[2];
    float cthr[2], ctest[2], gbound[2], dmin[2];
    int cpos[2], ccount[2], cpub[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int slot = slot0 + 32 * qb;
        qvalid[qb] = slot < a.nq;
        qidx[qb] = a.qlist ? a.qlist[qvalid[qb] ? slot : 0] : (qvalid[qb] ? slot : 0);
        // threshold key (nothing passes -inf: padding slots) and position (equal keys pass
        // at positions <= cpos)
        cthr[qb] = -kInf;
        cpos[qb] = -1;
        if (qvalid[qb]) {
            cthr[qb] = from_total_key(a.thr_key[qidx[qb]]);
            cpos[qb] = a.thr_pos[qidx[qb]];
        }
        gbound[qb] = kInf;  // DYN: the shared bound as last refreshed
        ctest[qb] = cthr[qb];  // min(cthr, gbound): pre-screen of the key tests
        dmin[qb] = kInf;
        ccount[qb] = 0;
        cpub[qb] = kTotalKeyInf;  // DYN: this lane's published running minimum
    }
    int next_refresh = 0;  // DYN: tile index of the next refresh
    // DYN: the largest D of the split's tiles tested so far, a block (its key f D is the
    // running minimum a lane publishes)
    float vmax0 = -kInf, vmax1 = -kInf;
    // the block's query's shared-bound slots: slot s at gbest_of(qb)[s * gbest_ld]
    auto gbest_of = [&](int qb) __attribute__((always_inline)) {
        return a.gbest + opaque(qidx[qb]);
    };
    // this lane's region of block qb: [slot][split][h][cap]
    auto region_of = [&](int qb) __attribute__((always_inline)) {
        return (((int64_t)opaque(slot0 + 32 * qb) * a.splits + split) * 2 + h) * a.cap;
    };

    // one row at or below block qb's pre-screen (d: its D): the exact test of its key and the
    // append. Past the region's capacity the count still grows (the select sees the
    // overflow); with cand_dmin the region keeps its first cap rows and dmin the smallest
    // key of the rows it drops, else the last slot is rewritten.
    auto test_row = [&](auto qb_tag, float d, int pos) __attribute__((always_inline)) {
        constexpr int qb = decltype(qb_tag)::value;
        const float kv = kF * d;
        if (((kv < cthr[qb]) | ((kv == cthr[qb]) & (pos <= cpos[qb]))) & (kv <= gbound[qb])) {
            PX_DCHECK(a.dbg, kDbgCollect, qvalid[qb] && pos >= row0 && pos < row1);
            if (ccount[qb] < a.cap || !a.cand_dmin) {
                const int64_t at = region_of(qb) + min(ccount[qb], a.cap - 1);
                a.cand_keys[at] = kv;
                a.cand_pos[at] = pos;
            } else {
                dmin[qb] = fminf(dmin[qb], kv);
            }
            ++ccount[qb];
        }
    };
    using Q0 = std::integral_constant<int, 0>;
    using Q1 = std::integral_constant<int, 1>;
    // key = f D (L2: ||x||^2 - 2 q.x, without the per-query ||q||^2, which does not change a
    // query's order, the select re-ranking exactly; IP: -q.x); a key is at or below ctest
    // exactly when D is at or above nct = ctest / f
    auto nct_of = [&](int qb) __attribute__((always_inline)) { return ctest[qb] * (1.0f / kF); };
    float nct[2] = {nct_of(0), nct_of(1)};
    // DYN, a split's first tile (keys in place): its kl-th smallest key bounds the split,
    // taken where some query of the wave has no threshold
    auto first_tile_bound = [&](f32x16 (&acc)[2], int rem) __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            if (__ballot(qvalid[qb] && cthr[qb] == kInf)) {
                gbound[qb] =
                    fminf(gbound[qb], first_tile_kth16(acc[qb], kF, rem, qvalid[qb], a.kl));
                ctest[qb] = fminf(cthr[qb], gbound[qb]);
                nct[qb] = nct_of(qb);
            }
        }
    };

    // the queries (MFMA B operands): dims 16 g + 8 h .. + 7 of each block's query, fp16;
    // padding slots load query 0's row and are never tested
    f16x8 b0[NG], b1[NG];
    {
        const unsigned short* q0h = a.queries_h + (int64_t)qidx[0] * kChunk + h * 8;
        const unsigned short* q1h = a.queries_h + (int64_t)qidx[1] * kChunk + h * 8;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            b0[g] = *reinterpret_cast<const f16x8*>(q0h + g * 16);
            b1[g] = *reinterpret_cast<const f16x8*>(q1h + g * 16);
        }
    }

    f32x16 accA[2], accB[2];
    // A operand of row j of a stage buffer's tile sub: the lane's 16 bytes of a dim group
    auto tile_at = [&](int buf, int sub) __attribute__((always_inline)) {
        return tile[buf] + (sub * kTile16 + j) * kPitch16 + h * 16;
    };
    // L2: tile t's accumulator starts, -||x||^2 / 2 of its rows in the MFMA result's layout
    // (acc[x]: row mfma_row(x, h), so four contiguous values a 4-register group), the same for
    // both query blocks. Read a tile ahead into the set the tile will use (it holds nothing
    // live by then); the lane offset is opaque so that each block's copy is its own LDS
    // read rather than one read and sixteen register copies.
    auto load_start = [&](int t, f32x16 (&acc)[2]) __attribute__((always_inline)) {
        if constexpr (L2) {
            const float* slot = tnorm[t & (kNormSlots16 - 1)];
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                const float* tn = slot + opaque(4 * h);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float4 v = *reinterpret_cast<const float4*>(tn + 8 * m);
                    acc[qb][4 * m + 0] = v.x;
                    acc[qb][4 * m + 1] = v.y;
                    acc[qb][4 * m + 2] = v.z;
                    acc[qb][4 * m + 3] = v.w;
                }
            }
        }
    };
    f16x8 an = *reinterpret_cast<const f16x8*>(tile_at(0, 0));  // the next tile's group 0
    load_start(0, accA);
    int rb_cur = 0;  // LDS buffer of the current stage
    int s = 0;       // stage index

    // One tile t (sub = t % 4 of stage s): its MFMAs into cur; TEST (t > 0): tile t - 1's D
    // values, in prev, tested between them. sub 0 begins the stage (its global loads); sub 3,
    // or the split's last tile, ends it (the sync and commit).
    auto run_tile = [&](auto test_tag, auto first_tag, auto sub_tag, int t, f32x16 (&cur)[2],
                        f32x16 (&prev)[2], auto whole_tag) __attribute__((always_inline)) {
        constexpr bool TEST = decltype(test_tag)::value;
        constexpr int SUB = decltype(sub_tag)::value;
        constexpr bool WHOLE = decltype(whole_tag)::value;  // tile t + 1 is in this stage
        const int rb_nxt = rb_cur == kBufs16 - 1 ? 0 : rb_cur + 1;
        const int rb_wr = rb_nxt == kBufs16 - 1 ? 0 : rb_nxt + 1;
        if constexpr (SUB == 0) {
            fetch();
            stage_ids(s + 3);
        }
        // DYN, the split's first tile (FIRST: t == 1): its own bound before its tests
        constexpr bool first = DYN && TEST && decltype(first_tag)::value;
        if constexpr (first) first_tile_bound(prev, kTile16);
        const int pt0 = row0 + (t - 1) * kTile16;  // first position of tile t - 1
        const char* ta = tile_at(rb_cur, SUB);
        // A operands are read two groups ahead (xa: group g + 1, xb: g + 2)
        f16x8 xa = an, xb = *reinterpret_cast<const f16x8*>(ta + 32);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const f16x8 x = xa;
            xa = xb;
            if (g + 2 < NG) xb = *reinterpret_cast<const f16x8*>(ta + (g + 2) * 32);
            if (g == 0 && !L2) {
                cur[0] = mfma16z(x, b0[0]);
                cur[1] = mfma16z(x, b1[0]);
            } else {
                cur[0] = mfma16(x, b0[g], cur[0]);
                cur[1] = mfma16(x, b1[g], cur[1]);
            }
            if constexpr (TEST) {
                // D 4 m .. 4 m + 3 (m = g % 4) of block g / 4: rows 8 m + 4 h .. + 3; the
                // group's largest against nct (the tests are rare: the branch falls through)
                const int r = 4 * (g & 3);
                const f32x16& pv = g < 4 ? prev[0] : prev[1];
                float dv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) dv[e] = pv[r + e];
                const float dmax = max_raw(max3_raw(dv[0], dv[1], dv[2]), dv[3]);
                if (g < 4) {
                    if constexpr (DYN) vmax0 = max_raw(vmax0, dmax);
                    if (__builtin_expect(__ballot(dmax >= nct[0]) != 0, 0)) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) test_row(Q0{}, dv[e], pt0 + mfma_row(r + e, h));
                    }
                } else {
                    if constexpr (DYN) vmax1 = max_raw(vmax1, dmax);
                    if (__builtin_expect(__ballot(dmax >= nct[1]) != 0, 0)) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) test_row(Q1{}, dv[e], pt0 + mfma_row(r + e, h));
                    }
                }
            }
        }
        // the LDS commit stays after the MFMAs: the scheduler would otherwise hoist it (to
        // shorten the prefetch registers' lives) and wait for the global loads there
        __builtin_amdgcn_sched_barrier(0);
        // DYN, on a doubling schedule of tiles (t - 1 = 0, 1, 2, 4, 8, ...): each block's
        // running minimum published (after this tile's commit) where it improved, and the
        // bound refreshed from the 32 published slots, whose kl-th smallest bounds the best kl.
        // Between those tiles only the running maxima are kept (one instruction a group):
        // publishing every tile measured slower, the vector instructions being the bound.
        bool pub0 = false, pub1 = false;
        bool refreshed = false;  // uniform: only a refresh tile publishes
        if constexpr (TEST && DYN) {
            if (t - 1 == next_refresh) {
                refreshed = true;
                const int tk0 = total_key(kF * vmax0), tk1 = total_key(kF * vmax1);
                pub0 = qvalid[0] && tk0 < cpub[0];
                pub1 = qvalid[1] && tk1 < cpub[1];
                cpub[0] = pub0 ? tk0 : cpub[0];
                cpub[1] = pub1 ? tk1 : cpub[1];
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    int v[16];
                    load_slots16(gbest_of(qb), a.gbest_ld, h, v);
                    gbound[qb] = fminf(gbound[qb], from_total_key(kth_smallest32(v, a.kl)));
                    ctest[qb] = fminf(cthr[qb], gbound[qb]);
                    nct[qb] = nct_of(qb);
                }
                next_refresh = (t - 1) + max(1, t - 1);
            }
        }
        auto publish_minima = [&]() __attribute__((always_inline)) {
            if constexpr (DYN) {
                if (refreshed) {
                    if (pub0) atomicMin(gbest_of(0) + (int64_t)(split & 31) * a.gbest_ld, cpub[0]);
                    if (pub1) atomicMin(gbest_of(1) + (int64_t)(split & 31) * a.gbest_ld, cpub[1]);
                }
            }
        };
        if constexpr (SUB < kTilesPerStage16 - 1) {
            if (WHOLE || t + 1 < ntiles) {
                // the stage's next tile: its first A operand and accumulator starts from the
                // same buffer, no sync
                an = *reinterpret_cast<const f16x8*>(tile_at(rb_cur, SUB + 1));
                load_start(t + 1, prev);
                publish_minima();
                return;
            }
        }
        // the next stage's first A operand and accumulator starts, and this wave's part of
        // stage s + 2, once every wave has committed stage s + 1
        wait_committed(s + 1);
        pair_priority(__hip_atomic_load(committed + (wave ^ 4), __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_WORKGROUP),
                      s + 1);
        if (s + 1 < nstages) {
            an = *reinterpret_cast<const f16x8*>(tile_at(rb_nxt, 0));
            load_start(t + 1, prev);
        }
        commit(s + 2, rb_wr);
        stage_publish(committed, wave, lane, s + 2);
        // published after the commit, whose waits then do not wait for the atomics
        publish_minima();
        rb_cur = rb_nxt;
        ++s;
    };
    using T = std::true_type;
    using F = std::false_type;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    // stage 0 (tile 1 tests tile 0, the split's first), then whole stages
    run_tile(F{}, F{}, S0{}, 0, accA, accB, F{});
    if (ntiles > 1) run_tile(T{}, T{}, S1{}, 1, accB, accA, F{});
    if (ntiles > 2) run_tile(T{}, F{}, S2{}, 2, accA, accB, F{});
    if (ntiles > 3) run_tile(T{}, F{}, S3{}, 3, accB, accA, F{});
    // whole stages, then the split's last (partial) one with its per-tile checks
    int tw = 4;
    for (; tw + 4 <= ntiles; tw += 4) {
        run_tile(T{}, F{}, S0{}, tw, accA, accB, T{});
        run_tile(T{}, F{}, S1{}, tw + 1, accB, accA, T{});
        run_tile(T{}, F{}, S2{}, tw + 2, accA, accB, T{});
        run_tile(T{}, F{}, S3{}, tw + 3, accB, accA, F{});
    }
    if (tw < ntiles) {
        run_tile(T{}, F{}, S0{}, tw, accA, accB, F{});
        if (tw + 1 < ntiles) run_tile(T{}, F{}, S1{}, tw + 1, accB, accA, F{});
        if (tw + 2 < ntiles) run_tile(T{}, F{}, S2{}, tw + 2, accA, accB, F{});
    }

    // the last tile's D values: all tested at once, with no MFMAs to hide behind
    auto finish = [&](f32x16 (&acc)[2]) __attribute__((always_inline)) {
        const int tl = ntiles - 1;
        const int t0 = row0 + tl * kTile16;
        const int rem = min(row1 - t0, kTile16);
        if constexpr (DYN) {
            if (tl == 0) first_tile_bound(acc, rem);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                // the split's running maximum with the last tile's rows
                float vmax = qb == 0 ? vmax0 : vmax1;
#pragma unroll
                for (int x = 0; x < 16; ++x)
                    vmax = mfma_row(x, h) < rem ? fmaxf(vmax, acc[qb][x]) : vmax;
                const int tk = total_key(kF * vmax);
                if (qvalid[qb] && tk < cpub[qb])
                    atomicMin(gbest_of(qb) + (int64_t)(split & 31) * a.gbest_ld, tk);
            }
        }
#pragma unroll
        for (int x = 0; x < 16; x += 2) {
            const int o0 = mfma_row(x, h), o1 = mfma_row(x + 1, h);
            {
                const float d0 = acc[0][x], d1 = acc[0][x + 1];
                if (__ballot((o0 < rem && d0 >= nct[0]) || (o1 < rem && d1 >= nct[0]))) {
                    if (o0 < rem) test_row(Q0{}, d0, t0 + o0);
                    if (o1 < rem) test_row(Q0{}, d1, t0 + o1);
                }
            }
            {
                const float d0 = acc[1][x], d1 = acc[1][x + 1];
                if (__ballot((o0 < rem && d0 >= nct[1]) || (o1 < rem && d1 >= nct[1]))) {
                    if (o0 < rem) test_row(Q1{}, d0, t0 + o0);
                    if (o1 < rem) test_row(Q1{}, d1, t0 + o1);
                }
            }
        }
    };
    if (ntiles & 1) finish(accA);
    else finish(accB);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        if (qvalid[qb]) {
            const int64_t r = ((int64_t)(slot0 + 32 * qb) * a.splits + split) * 2 + h;
            a.cand_count[r] = ccount[qb];
            if (a.cand_dmin && ccount[qb] > a.cap) a.cand_dmin[r] = total_key(dmin[qb]);
        }
    }
}

}  // namespace

int flat_collect16_queries_per_block() { return kQueriesPerBlock16; }

hipError_t launch_flat_collect16(const FlatScanArgs& a, hipStream_t s) {
    if (a.dp != kChunk || a.dense || !a.corpus_h || !a.queries_h) return hipErrorInvalidValue;
    const bool dyn = a.gbest != nullptr;
    const int64_t qtiles = (a.nq + kQueriesPerBlock16 - 1) / kQueriesPerBlock16;
    const dim3 grid((unsigned)(qtiles * a.splits)), block(512);
    const FlatScanArgs b = with_spin_limit(a);
#define PX_COLLECT16(L2, FILT, DYN) \
    hipLaunchKernelGGL((flat_collect16_kernel<L2, FILT, DYN>), grid, block, 0, s, b)
    if (a.metric == 0) {
        if (a.rowidx) {
            if (dyn) PX_COLLECT16(true, true, true);
            else PX_COLLECT16(true, true, false);
        } else if (dyn) PX_COLLECT16(true, false, true);
        else PX_COLLECT16(true, false, false);
    } else {
        if (a.rowidx) {
            if (dyn) PX_COLLECT16(false, true, true);
            else PX_COLLECT16(false, true, false);
        } else if (dyn) PX_COLLECT16(false, false, true);
        else PX_COLLECT16(false, false, false);
    }
#undef PX_COLLECT16
    return hipGetLastError();
}

}  // namespace px
