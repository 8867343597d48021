// px_collect.hip -- the threshold-collect scan of FlatIndex searches for gfx950.
//
// Replaces the per-query full scan of crates/core/src/flat.rs:106-148 on the collect path
// (large k, moderate k on large batches, and the bounded first round of the 1M x 128
// workload): every row whose MFMA key (||x||^2 - 2 q.x for L2, -q.x for IP) is at or below
// its query's threshold is appended to a candidate region; flat_collect_select_kernel
// re-ranks the best k + 8 in the reference's arithmetic (distance.rs:3-39) and finishes.
//
// One workgroup = 8 waves = 256 queries (each wave: 32 queries' fragments in registers as
// the MFMA B operand) x one corpus split. The corpus streams through LDS in stages of 64
// rows x 128 dims (one tile is ceil(dp / 128) stages).
//
// Pipeline. Three LDS stage buffers: stage s reads buffer s % 3 while the global loads of
// stage s + 2 are in flight in registers; they are written to buffer (s + 2) % 3 after the
// stage's MFMAs. There is no barrier per stage: each wave publishes in LDS the last stage
// it has committed, and at the end of stage s waits until every wave has committed stage
// s + 1; then it reads the A operands of stage s + 1's first dim group, writes its part of
// stage s + 2, and issues stage s + 1's first MFMAs, at most one stage ahead of the slowest
// wave of its workgroup. Two accumulator sets alternate between tiles: while the MFMAs of
// tile t accumulate into one set, the keys of tile t - 1 are computed from the other, in
// place, and tested against the thresholds two rows per dim group, between the MFMAs of
// tile t's first stage; so no wave leaves the matrix unit idle for an epilogue. Each
// tile's row norms (L2) sit in one of four small LDS buffers, kept until its keys are
// computed a tile later.
//
// H16 (FlatScanArgs::corpus_h / queries_h: rows and queries whose every value is exact in
// fp16): the same scan on v_mfma_f32_32x32x16_f16 with fp32 accumulation. Each product is
// exact in fp16 as in fp32, so the keys are the fp32 scan's up to the rounding of the sums.
// A group of 16 dims is only two MFMAs, so a stage holds two tiles (one stage sync per 32
// MFMAs of a wave), norms sit in eight slots (one a tile), and each group's A operands and
// norms are read two groups ahead. Here it serves the dense keys of a threshold sample
// only: thresholded and bounded fp16 scans run in px_collect16.hip (64 queries a wave).
//
// Appends go to one of two regions per (query slot, split), one per lane of the pair that
// holds the query (lanes l and l ^ 32 hold the two halves of the query's 64 rows of a
// tile), each with its own counter, so appends need no cross-lane step. dense: no
// thresholds; every key of the split is written to cand_keys [slot][dense_ld] by position
// (the threshold sample of the sampled path).
//
// DYN (one-chunk scans with FlatScanArgs::gbest, filtered or not): the splits' shared bound.
// After each tile a lane publishes the smallest key of its rows of the split so far to
// slot split % 32 of its query (device-scope atomicMin: a plain store would stay in this
// XCD's L2); every published slot then has a row of its own splits at or below it, so the
// kl-th smallest slot bounds the query's best kl, and rows above it are not appended.
// The bound is refreshed on a geometric schedule of tiles (t -> t + t/2); the refresh's
// loads are issued at the start of a stage and consumed after its MFMAs. A split's first
// tile also bounds itself by its own kl-th smallest key (so a query needs no threshold).
#include "px_device.h"
#include "px_kernels.h"
#include "px_scan_common.h"

#include <float.h>

#include <type_traits>

namespace px {

namespace {

constexpr int kStageBufs = 3;  // LDS stage buffers
constexpr int kNormBufs = 4;   // LDS norm buffers (tile t + 2 is staged while t - 1 is tested)

template <bool L2, bool MULTI, bool FILT, bool DYN, bool FULL, bool H16>
__global__ __launch_bounds__(512) void flat_collect_kernel(FlatScanArgs a) {
    constexpr int NT = 512;
    // H16: rows and queries as fp16 (FlatScanArgs::corpus_h, queries_h), 16 dims a MFMA;
    // a staged row is 256 bytes (else 512), its LDS pitch 16 bytes more (conflict-free b128
    // reads: sixteen consecutive rows' same piece fall in sixteen different bank groups)
    constexpr int kRowBytes = H16 ? kChunk * 2 : kChunk * 4;
    constexpr int kPitch = kRowBytes + 16;
    constexpr int kF4PerRow = kRowBytes / 16;    // 16-byte pieces per staged row (32; H16 16)
    constexpr int kRowStep = NT / kF4PerRow;     // rows between a thread's loads (16; H16 32)
    // H16: a stage is two tiles (128 rows), so that the stage sync is paid once per 32 MFMAs
    // of a wave, as on fp32 it is once per 128
    constexpr int TPS = H16 ? 2 : 1;             // tiles per stage
    constexpr int kStageRows = TPS * kTileRows;
    constexpr int kPF = kStageRows / kRowStep;   // pieces per thread per stage (4)
    constexpr int NG = H16 ? 8 : 16;             // MFMA dim groups per 128-dim chunk
    constexpr int KPG = 32 / NG;                 // keys of the previous tile tested per group
    constexpr int kNB = H16 ? 8 : kNormBufs;     // norm slots (one a tile)
    constexpr int kBufFloats = H16 ? kStageRows * kPitch / 4 : kTileRows * kLdsStride;
    static_assert(NT % kF4PerRow == 0 && kStageRows % kRowStep == 0, "uneven stage split");
    static_assert(!(H16 && MULTI), "fp16 rows are one 128-dim chunk");
    static_assert(H16 || kPitch == kLdsStride * 4, "fp32 rows keep the list scan's pitch");
    static_assert(!(DYN && MULTI), "the shared bound serves one-chunk scans");
    __shared__ __attribute__((aligned(16))) float tile[kStageBufs][kBufFloats];
    __shared__ __attribute__((aligned(16))) float tnorm[kNB][kTileRows];
    // per wave: the last stage it has committed to a stage buffer (the stage sync below)
    __shared__ int committed[8];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    // query tiles in reverse launch order: the last (partial) tile, whose workgroups run
    // fastest, starts in the first round of workgroups with all its splits together, so
    // none of them scans far ahead of the others' shared bound
    const int qtiles = gridDim.x / a.splits;
    const int qt = qtiles - 1 - (int)(blockIdx.x / a.splits), split = blockIdx.x % a.splits;
    const int slot = qt * 256 + wave * 32 + j;
    const bool qvalid = slot < a.nq;
    const int q = a.qlist ? a.qlist[qvalid ? slot : 0] : slot;
    // positions, tiles and stages fit 32 bits (at most 2^31 - 2 rows; host-checked)
    const int row0 = (int)((int64_t)split * a.rows_per_split);
    const int row1 = (int)min(a.n_eff, (int64_t)row0 + a.rows_per_split);
    PX_DCHECK(a.dbg, kDbgCollect, row0 < row1 && (int64_t)qtiles * a.splits == (int64_t)gridDim.x);
    const float kInf = __int_as_float(0x7f800000);
    const int nch = MULTI ? (a.dp + kChunk - 1) / kChunk : 1;
    const int ntiles = (row1 - row0 + kTileRows - 1) / kTileRows;  // >= 1
    const int nstages = MULTI ? ntiles * nch : (ntiles + TPS - 1) / TPS;
    const int cc = tid % kF4PerRow;   // this thread's float4 column of a staged row
    const int rr0 = tid / kF4PerRow;  // its first row of a stage

    // ---- staging: row ids, global loads held in registers, commit to LDS ----------------
    // Every load is unconditional with a clamped address (rows past the split's end read
    // row 0, columns past a chunk's end repeat its last float4): such rows' keys are never
    // tested or are written as +inf, and such columns are never multiplied (dim groups
    // past the chunk's end are skipped).
    int rid[kPF], pid;
    // (positions past the split's end are formed in 64 bits: near 2^31 rows they overflow)
    auto tile_ids = [&](int t) __attribute__((always_inline)) {  // t: a stage's first tile / TPS
        const int64_t t0 = (int64_t)row0 + (int64_t)t * kStageRows;
#pragma unroll
        for (int u = 0; u < kPF; ++u) {
            const int64_t pos = t0 + rr0 + u * kRowStep;
            const int v = FILT ? a.rowidx[min(pos, (int64_t)row1 - 1)] : (int)pos;
            rid[u] = pos < row1 ? v : -1;
            PX_DCHECK(a.dbg, kDbgCollect, pos >= row1 || (v >= 0 && v < a.rows));
        }
        const int64_t pos = t0 + tid;
        const int v = FILT ? a.rowidx[min(pos, (int64_t)row1 - 1)] : (int)pos;
        pid = (tid < kStageRows && pos < row1) ? v : -1;
    };
    static_assert(kPF == 4, "four staged pieces per thread");
    float4 pf0, pf1, pf2, pf3;  // separate variables: an array of them ended up in memory
    float pn = 0.f;
    auto fetch = [&](int s) __attribute__((always_inline)) {
        const int c = MULTI ? (int)(s % nch) : 0;
        if constexpr (H16) {
            const unsigned short* base = a.corpus_h + cc * 8;
            pf0 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[0], 0) * kChunk);
            pf1 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[1], 0) * kChunk);
            pf2 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[2], 0) * kChunk);
            pf3 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[3], 0) * kChunk);
        } else {
            const int f4r = min(kChunk, a.dp - c * kChunk) >> 2;
            const float* base = a.corpus + c * kChunk + min(cc, f4r - 1) * 4;
            pf0 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[0], 0) * a.dp);
            pf1 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[1], 0) * a.dp);
            pf2 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[2], 0) * a.dp);
            pf3 = *reinterpret_cast<const float4*>(base + (int64_t)max(rid[3], 0) * a.dp);
        }
        if (L2 && c == 0) pn = a.norms[max(pid, 0)];
    };
    auto commit = [&](int s, int buf) __attribute__((always_inline)) {
        char* tb = reinterpret_cast<char*>(tile[buf]) + rr0 * kPitch + cc * 16;
        *reinterpret_cast<float4*>(tb) = pf0;
        *reinterpret_cast<float4*>(tb + kRowStep * kPitch) = pf1;
        *reinterpret_cast<float4*>(tb + 2 * kRowStep * kPitch) = pf2;
        *reinterpret_cast<float4*>(tb + 3 * kRowStep * kPitch) = pf3;
        if constexpr (H16) {
            // the stage's two tiles' norms, one slot a tile
            if (L2 && tid < kStageRows) tnorm[(TPS * s + (tid >> 6)) & (kNB - 1)][tid & 63] = pn;
        } else {
            const int c = MULTI ? (int)(s % nch) : 0;
            if (L2 && c == 0 && tid < kTileRows) tnorm[(s / nch) & (kNormBufs - 1)][tid] = pn;
        }
    };

    // prologue: stages 0 and 1 in LDS, ids of the tile of stage 2
    tile_ids(0);
    fetch(0);
    commit(0, 0);
    tile_ids(1 / nch);
    fetch(1);
    commit(1, 1);
    tile_ids(2 / nch);
    if (tid < 8) committed[tid] = 1;
    __syncthreads();

    // Stage sync without a barrier per stage. The two waves of a SIMD do not finish a
    // stage's MFMAs together (the matrix unit favours one), and at a workgroup barrier the
    // one ahead would idle while the other finishes and commits; with three stage buffers a
    // wave may instead run up to a stage ahead. Each wave publishes the last stage it has
    // committed (committed[wave], an LDS store with release order), and at the end of stage
    // s waits until every wave has committed stage s + 1 (acquire loads) before it reads
    // stage s + 1's buffer and writes stage s + 2's. A wave commits stage s + 1 only after
    // all its reads of stage s - 1, whose buffer and norm slot the writes of stage s + 2
    // reuse, so the one wait covers both. A wait gives up after a.spin_limit polls
    // (kSpinLimit, about 5 ms, unless a test lowers it) and reports it (a.spin_fail), so
    // that a wave always finishes.
    auto publish = [&](int v) __attribute__((always_inline)) {
        stage_publish(committed, wave, lane, v);
    };
    const unsigned caddr = (unsigned)(uintptr_t)(committed + (lane & 7));
    auto wait_committed = [&](int ct) __attribute__((always_inline)) {
        if (stage_wait(caddr, ct, a.spin_limit) >= a.spin_limit && a.spin_fail && lane == 0)
            atomicOr(a.spin_fail, 1);
    };

    // A wave whose 32 queries are all padding (last query tile) only helps stage the
    // corpus: same loads, same waits.
    if (qt * 256 + wave * 32 >= a.nq) {
        int wb = 2;
        for (int s = 0; s < nstages; ++s) {
            fetch(s + 2);
            tile_ids((s + 3) / nch);
            wait_committed(s + 1);
            commit(s + 2, wb);
            publish(s + 2);
            wb = wb == kStageBufs - 1 ? 0 : wb + 1;
        }
        return;
    }

    // ---- per-query state ----------------------------------------------------------------
    float cthr = -kInf;  // threshold key (nothing passes -inf: padding slots, dense mode)
    int cpos = -1;       // threshold position (equal keys pass at positions <= cpos)
    if (qvalid && !a.dense) {
        cthr = from_total_key(a.thr_key[q]);
        cpos = a.thr_pos[q];
    }
    float gbound = kInf;  // DYN: the shared bound as last refreshed
    float ctest = cthr;   // min(cthr, gbound): pre-screen of the key tests
    int ccount = 0;       // rows appended (or counted past the region's capacity)
    int* gbest = DYN ? a.gbest + (qvalid ? q : 0) : nullptr;  // slot s at gbest[s * gbest_ld]
    int cpub = kTotalKeyInf;     // DYN: this lane's published running minimum
    int next_refresh = 0;        // DYN: tile index of the next refresh
    float* const creg_k = a.cand_keys + ((int64_t)slot * a.splits + split) * 2 * a.cap +
                          (int64_t)h * a.cap;
    int* const creg_p = a.cand_pos + ((int64_t)slot * a.splits + split) * 2 * a.cap +
                        (int64_t)h * a.cap;

    // one row of the previous tile at or below the pre-screen: the exact test and append.
    // Past the region's capacity the count still grows (the select sees the overflow). With
    // cand_dmin the region keeps its first cap rows and dmin the smallest key of the rows
    // it drops (the select finishes a query whose k'-th kept key is below every dropped
    // key); without it the last slot is rewritten.
    float dmin = kInf;
    auto test_row = [&](float kv, int pos) __attribute__((always_inline)) {
        if (((kv < cthr) | ((kv == cthr) & (pos <= cpos))) & (kv <= gbound)) {
            PX_DCHECK(a.dbg, kDbgCollect, qvalid && pos >= row0 && pos < row1);
            if (ccount < a.cap || !a.cand_dmin) {
                const int at = min(ccount, a.cap - 1);
                creg_k[at] = kv;
                creg_p[at] = pos;
            } else {
                dmin = fminf(dmin, kv);
            }
            ++ccount;
        }
    };
    // keys of a tile from its accumulators, in place: key[x] is row
    // 32 (x / 16) + mfma_row(x % 16, h) of the tile; L2 drops the per-query ||q||^2 (it does
    // not change a query's order, and the select re-ranks exactly), IP negates
    auto key_of = [&](float dot, float nrm) __attribute__((always_inline)) {
        return L2 ? __builtin_fmaf(-2.0f, dot, nrm) : -dot;
    };
    auto all_keys = [&](f32x16 (&acc)[2], const float* tn) __attribute__((always_inline)) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int m4 = 0; m4 < 4; ++m4) {
                float4 nv = make_float4(0.f, 0.f, 0.f, 0.f);
                if (L2) nv = *reinterpret_cast<const float4*>(tn + rb * 32 + 8 * m4 + 4 * h);
                acc[rb][4 * m4 + 0] = key_of(acc[rb][4 * m4 + 0], nv.x);
                acc[rb][4 * m4 + 1] = key_of(acc[rb][4 * m4 + 1], nv.y);
                acc[rb][4 * m4 + 2] = key_of(acc[rb][4 * m4 + 2], nv.z);
                acc[rb][4 * m4 + 3] = key_of(acc[rb][4 * m4 + 3], nv.w);
            }
    };
    auto as_keys = [](f32x16 (&acc)[2], float (&k)[32]) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < 32; ++x) k[x] = acc[x >> 4][x & 15];
    };
    // every key of a tile, row-major by position (+inf past the split's end), so that each
    // query's keys are contiguous for the ladder: keys 4 m .. 4 m + 3 of a lane are four
    // consecutive rows
    auto dense_write = [&](f32x16 (&acc)[2], int t0, int rem) __attribute__((always_inline)) {
        if (!qvalid) return;
        PX_DCHECK(a.dbg, kDbgCollect, t0 >= 0 && (int64_t)t0 + kTileRows <= a.dense_ld);
        float* dst = a.cand_keys + (int64_t)slot * a.dense_ld + t0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int x = 4 * m + e;
                v[e] = (x >> 4) * 32 + mfma_row(x & 15, h) < rem ? acc[x >> 4][x & 15] : kInf;
            }
            const int lr = (m >> 2) * 32 + 8 * (m & 3) + 4 * h;
            *reinterpret_cast<float4*>(dst + lr) = make_float4(v[0], v[1], v[2], v[3]);
        }
    };
    // DYN, a split's first tile (keys in place): its kl-th smallest key bounds the split,
    // taken where some query of the wave has no threshold (a sampled one already bounds the
    // first tile far below)
    auto first_tile_bound = [&](f32x16 (&acc)[2], int rem) __attribute__((always_inline)) {
        if (__ballot(qvalid && cthr == kInf)) {
            float k[32];
            as_keys(acc, k);
            gbound = fminf(gbound, first_tile_kth(k, rem, qvalid, a.kl));
        }
    };

    // query chunk 0 (MFMA B operand): dims past the chunk's end are loaded clamped and never
    // multiplied; padding query slots load query 0's row and are never tested
    // (H16: dims 16 g + 8 h .. + 7 of the query, fp16)
    const float* qrow = a.queries + (int64_t)(qvalid ? q : 0) * a.dp;
    using Frag = std::conditional_t<H16, f16x8, float4>;  // one lane's operand of a dim group
    Frag b[NG];
    if constexpr (H16) {
        const unsigned short* qh = a.queries_h + (int64_t)(qvalid ? q : 0) * kChunk + h * 8;
#pragma unroll
        for (int g = 0; g < NG; ++g) b[g] = *reinterpret_cast<const f16x8*>(qh + g * 16);
    } else {
        const int dc = min(kChunk, a.dp);
#pragma unroll
        for (int g = 0; g < NG; ++g)
            b[g] = *reinterpret_cast<const float4*>(qrow + min(g * 8 + h * 4, dc - 4));
    }

    f32x16 accA[2], accB[2];
    // A operands of the next stage's first dim group (read at the end of each stage): rows
    // j and 32 + j, the lane's 16 bytes of a 32-byte dim group
    auto tile_at = [&](int buf, int row) __attribute__((always_inline)) {
        return reinterpret_cast<const char*>(tile[buf]) + row * kPitch + h * 16;
    };
    Frag an0 = *reinterpret_cast<const Frag*>(tile_at(0, j));
    Frag an1 = *reinterpret_cast<const Frag*>(tile_at(0, 32 + j));
    int rb_cur = 0;  // LDS buffer of the current stage
    int s = 0;       // stage index

    // One stage: the MFMAs of chunk c of tile t into cur. TEST (the first stage of tiles
    // t > 0): the keys of tile t - 1, in prev, computed and tested between them. H16 (two
    // tiles a stage): par_tag = t % 2; an even tile begins the stage (its loads), an odd
    // one (or the last tile) ends it (the sync and commit).
    auto stage = [&](auto test_tag, auto first_tag, auto par_tag, int t, int c,
                     f32x16 (&cur)[2], f32x16 (&prev)[2]) __attribute__((always_inline)) {
        constexpr bool TEST = decltype(test_tag)::value;
        constexpr bool BEGIN = !H16 || decltype(par_tag)::value == 0;
        const bool first = !MULTI || c == 0;
        const int rb_nxt = rb_cur == kStageBufs - 1 ? 0 : rb_cur + 1;
        const int rb_wr = rb_nxt == kStageBufs - 1 ? 0 : rb_nxt + 1;
        if constexpr (BEGIN) {
            fetch(s + 2);
            tile_ids((s + 3) / nch);
        }
        // DYN, the split's first tile (FIRST: t == 1): all its keys and its own bound before
        // its tests
        constexpr bool keys_ready = DYN && TEST && decltype(first_tag)::value;
        const float* tn = tnorm[(t - 1) & (kNB - 1)];
        if constexpr (keys_ready) {
            all_keys(prev, tn);
            first_tile_bound(prev, kTileRows);
            ctest = fminf(cthr, gbound);
        }
        const int pt0 = row0 + (t - 1) * kTileRows;  // first position of tile t - 1
        float vmin = kInf;  // DYN: smallest key of tile t - 1
        // dim groups of this chunk (FULL: dp is a multiple of 128, every chunk has all NG)
        const int ng = FULL ? NG : min(kChunk, a.dp - c * kChunk) >> 3;
        const int cn = MULTI ? (c + 1 == nch ? 0 : c + 1) : 0;
        const int dcn = min(kChunk, a.dp - cn * kChunk);
        constexpr int kRow0 = BEGIN ? 0 : kTileRows;  // the tile's first row in the stage
        const char* ta0 = tile_at(rb_cur, kRow0 + j);
        const char* ta1 = tile_at(rb_cur, kRow0 + 32 + j);
        float4 nv = make_float4(0.f, 0.f, 0.f, 0.f);
        // H16 (two MFMAs a group, too few to cover an LDS read): each group's A operands and
        // norms are read two groups ahead (xa, nvn: group g + 1; xb, nvb: g + 2)
        Frag xa0 = an0, xa1 = an1, xb0 = an0, xb1 = an1;
        float4 nvn = make_float4(0.f, 0.f, 0.f, 0.f), nvb = nvn;
        if constexpr (H16) {
            xb0 = *reinterpret_cast<const Frag*>(ta0 + 32);
            xb1 = *reinterpret_cast<const Frag*>(ta1 + 32);
            if constexpr (TEST && L2) {
                if (!keys_ready) {
                    nvn = *reinterpret_cast<const float4*>(tn + 4 * h);
                    nvb = *reinterpret_cast<const float4*>(tn + 8 + 4 * h);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            if (g < ng) {
                Frag x0, x1;
                if constexpr (H16) {
                    x0 = xa0;
                    x1 = xa1;
                    xa0 = xb0;
                    xa1 = xb1;
                    if (g + 2 < NG) {
                        xb0 = *reinterpret_cast<const Frag*>(ta0 + (g + 2) * 32);
                        xb1 = *reinterpret_cast<const Frag*>(ta1 + (g + 2) * 32);
                    }
                } else {
                    x0 = g == 0 ? an0 : *reinterpret_cast<const Frag*>(ta0 + g * 32);
                    x1 = g == 0 ? an1 : *reinterpret_cast<const Frag*>(ta1 + g * 32);
                }
                if (g == 0 && first) {
                    cur[0] = mfma_group_z(x0, b[0]);
                    cur[1] = mfma_group_z(x1, b[0]);
                } else {
                    cur[0] = mfma_group(x0, b[g], cur[0]);
                    cur[1] = mfma_group(x1, b[g], cur[1]);
                }
            }
            if constexpr (MULTI)
                b[g] = *reinterpret_cast<const float4*>(qrow + cn * kChunk +
                                                        min(g * 8 + h * 4, dcn - 4));
            if constexpr (TEST) {
                // rows x = KPG g .. KPG g + KPG - 1 of tile t - 1: block rb = x / 16, MFMA
                // rows r .. r + KPG - 1
                const int rb = (KPG * g) >> 4, r = (KPG * g) & 15;
                if (!keys_ready) {
                    if constexpr (H16) {
                        // rows 4g .. 4g + 3: norms at 8 g + 4 h (rb = g / 4, r = 4 (g % 4))
                        if (L2) {
                            nv = nvn;
                            nvn = nvb;
                            if (g + 2 < NG)
                                nvb = *reinterpret_cast<const float4*>(tn + 8 * (g + 2) + 4 * h);
                        }
                    } else if (L2 && (r & 3) == 0) {
                        nv = *reinterpret_cast<const float4*>(tn + rb * 32 + 8 * (r >> 2) + 4 * h);
                    }
                    const float nn[4] = {nv.x, nv.y, nv.z, nv.w};
#pragma unroll
                    for (int e = 0; e < KPG; ++e)
                        prev[rb][r + e] = key_of(prev[rb][r + e], nn[(r & 3) + e]);
                }
                // the group's smallest key decides whether any of its rows is tested (one
                // compare), and feeds the tile's minimum
                float kv[KPG];
#pragma unroll
                for (int e = 0; e < KPG; ++e) kv[e] = prev[rb][r + e];
                float kmin = kv[0];
#pragma unroll
                for (int e = 1; e < KPG; ++e) kmin = fminf(kmin, kv[e]);
                if constexpr (DYN) vmin = fminf(vmin, kmin);
                if (__ballot(kmin <= ctest)) {
#pragma unroll
                    for (int e = 0; e < KPG; ++e) test_row(kv[e], pt0 + rb * 32 + mfma_row(r + e, h));
                }
            }
        }
        // the stage's LDS commit stays after its MFMAs: the scheduler would otherwise hoist it
        // (to shorten the prefetch registers' lives) and wait for the global loads there
        __builtin_amdgcn_sched_barrier(0);
        bool pub_now = false;
        if constexpr (TEST) {
            if constexpr (DYN) {
                const int tk = total_key(vmin);
                pub_now = qvalid && tk < cpub;
                cpub = pub_now ? tk : cpub;
                if (t - 1 == next_refresh) {
                    // the query's 32 published slots; their kl-th smallest bounds its best kl
                    int v[16];
                    load_slots16(gbest, a.gbest_ld, h, v);
                    gbound = fminf(gbound, from_total_key(kth_smallest32(v, a.kl)));
                    next_refresh = (t - 1) + max(1, (t - 1) >> 1);
                }
                ctest = fminf(cthr, gbound);
            }
            if (a.dense) dense_write(prev, row0 + (t - 1) * kTileRows, kTileRows);
        }
        if (H16 && BEGIN && t + 1 < ntiles) {
            // the stage's second tile: its first A operands from the same buffer, no sync
            an0 = *reinterpret_cast<const Frag*>(tile_at(rb_cur, kTileRows + j));
            an1 = *reinterpret_cast<const Frag*>(tile_at(rb_cur, kTileRows + 32 + j));
            if constexpr (DYN) {
                if (pub_now) atomicMin(gbest + (int64_t)(split & 31) * a.gbest_ld, cpub);
            }
            return;
        }
        // the next stage's first A operands and this wave's part of stage s + 2, once every
        // wave has committed stage s + 1
        wait_committed(s + 1);
        pair_priority(__hip_atomic_load(committed + (wave ^ 4), __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_WORKGROUP),
                      s + 1);
        if (s + 1 < nstages) {
            an0 = *reinterpret_cast<const Frag*>(tile_at(rb_nxt, j));
            an1 = *reinterpret_cast<const Frag*>(tile_at(rb_nxt, 32 + j));
        }
        commit(s + 2, rb_wr);
        publish(s + 2);
        if constexpr (DYN) {
            // published after the commit, whose waits then do not wait for the atomic
            if (pub_now) atomicMin(gbest + (int64_t)(split & 31) * a.gbest_ld, cpub);
        }
        rb_cur = rb_nxt;
        ++s;
    };
    // a tile: its first stage tests the previous tile (TEST), its other chunks do not
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    auto run_tile = [&](auto test_tag, auto first_tag, auto par_tag, int t, f32x16 (&cur)[2],
                        f32x16 (&prev)[2]) __attribute__((always_inline)) {
        stage(test_tag, first_tag, par_tag, t, 0, cur, prev);
        for (int c = 1; c < nch; ++c)
            stage(std::false_type{}, std::false_type{}, par_tag, t, c, cur, prev);
    };
    // tile 0; tile 1 (its first stage tests tile 0, the split's first); then pairs
    run_tile(std::false_type{}, std::false_type{}, P0{}, 0, accA, accB);
    if (ntiles > 1) run_tile(std::true_type{}, std::true_type{}, P1{}, 1, accB, accA);
    for (int t = 2; t < ntiles; t += 2) {
        run_tile(std::true_type{}, std::false_type{}, P0{}, t, accA, accB);
        if (t + 1 < ntiles) run_tile(std::true_type{}, std::false_type{}, P1{}, t + 1, accB, accA);
    }

    // the last tile's keys: all at once, with no MFMAs to hide behind
    auto finish = [&](f32x16 (&acc)[2]) __attribute__((always_inline)) {
        const int tl = ntiles - 1;
        const int t0 = row0 + tl * kTileRows;
        const int rem = min(row1 - t0, kTileRows);
        all_keys(acc, tnorm[tl & (kNB - 1)]);
        if (a.dense) {
            dense_write(acc, t0, rem);
            return;
        }
        if constexpr (DYN) {
            if (tl == 0) {
                first_tile_bound(acc, rem);
                ctest = fminf(cthr, gbound);
            }
            float vmin = kInf;
#pragma unroll
            for (int x = 0; x < 32; ++x)
                vmin = (x >> 4) * 32 + mfma_row(x & 15, h) < rem ? fminf(vmin, acc[x >> 4][x & 15])
                                                                 : vmin;
            const int tk = total_key(vmin);
            if (qvalid && tk < cpub) atomicMin(gbest + (int64_t)(split & 31) * a.gbest_ld, tk);
        }
        const int pt0 = t0;
#pragma unroll
        for (int x = 0; x < 32; x += 2) {
            const float k0 = acc[x >> 4][x & 15], k1 = acc[x >> 4][(x & 15) + 1];
            const int o0 = (x >> 4) * 32 + mfma_row(x & 15, h);
            const int o1 = (x >> 4) * 32 + mfma_row((x & 15) + 1, h);
            if (__ballot((o0 < rem && k0 <= ctest) || (o1 < rem && k1 <= ctest))) {
                if (o0 < rem) test_row(k0, pt0 + o0);
                if (o1 < rem) test_row(k1, pt0 + o1);
            }
        }
    };
    if (ntiles & 1) finish(accA);
    else finish(accB);
    if (qvalid && !a.dense) {
        const int64_t r = ((int64_t)slot * a.splits + split) * 2 + h;
        a.cand_count[r] = ccount;
        if (a.cand_dmin && ccount > a.cap) a.cand_dmin[r] = total_key(dmin);
    }
}

}  // namespace

hipError_t launch_flat_collect(const FlatScanArgs& a, hipStream_t s) {
    // rows of exactly 128 padded dims (one full chunk: the 1M x 128 workload); rows of 129-384
    // take flat_list16q_kernel's collect mode (the queries resident in registers), except the
    // dense threshold-sample scans; other widths the collect mode of flat_scan_kernel
    if (a.dp != kChunk)
        return !a.dense && collect_resident_queries(a.dp) ? launch_flat_collect16q(a, s)
                                                          : launch_flat_collect_v1(a, s);
    const int64_t qtiles = (a.nq + 255) / 256;
    const dim3 grid((unsigned)(qtiles * a.splits)), block(512);
    const bool dyn = a.gbest != nullptr;
    if (dyn && a.dense) return hipErrorInvalidValue;
    if ((a.corpus_h == nullptr) != (a.queries_h == nullptr)) return hipErrorInvalidValue;
    const bool h16 = a.corpus_h != nullptr;
    // fp16 rows: thresholds or the shared bound take the 64-query-wave scan; the dense keys
    // of a threshold sample stay here
    if (h16 && !a.dense) return launch_flat_collect16(a, s);
    const FlatScanArgs b = with_spin_limit(a);
#define PX_COLLECT(L2, FILT, DYN)                                                              \
    do {                                                                                       \
        if constexpr (!(DYN)) {                                                                \
            if (h16) {                                                                         \
                hipLaunchKernelGGL((flat_collect_kernel<L2, false, FILT, false, true, true>),   \
                                   grid, block, 0, s, b);                                      \
                break;                                                                         \
            }                                                                                  \
        }                                                                                      \
        hipLaunchKernelGGL((flat_collect_kernel<L2, false, FILT, DYN, true, false>), grid,      \
                           block, 0, s, b);                                                    \
    } while (0)
    if (a.metric == 0) {
        if (a.rowidx) {
            if (dyn) PX_COLLECT(true, true, true);
            else PX_COLLECT(true, true, false);
        } else if (dyn) PX_COLLECT(true, false, true);
        else PX_COLLECT(true, false, false);
    } else {
        if (a.rowidx) {
            if (dyn) PX_COLLECT(false, true, true);
            else PX_COLLECT(false, true, false);
        } else if (dyn) PX_COLLECT(false, false, true);
        else PX_COLLECT(false, false, false);
    }
#undef PX_COLLECT
    return hipGetLastError();
}

}  // namespace px
