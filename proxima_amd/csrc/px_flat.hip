// px_flat.hip -- exact kNN (FlatIndex) kernels for gfx950.
//
// Replaces the per-query full scan of crates/core/src/flat.rs:106-148 (and the CUDA
// satellite crates/core/cuda/knn.cu:22-121) with a tiled fp32-MFMA contraction:
//   L2 key  = ||x||^2 + ||q||^2 - 2 q.x   (precomputed corpus norms in HBM)
//   IP key  = -q.x
// Corpus tiles of 64 rows are staged through LDS; each wave keeps 32 queries' fragments
// in registers (MFMA B operand) and a sorted candidate list per query in LDS, so the
// distance matrix never reaches HBM. Candidates are ordered by (key total-order, id).
// The split lists are merged by flat_merge_kernel, which re-ranks the survivors with the
// reference's exact arithmetic (distance.rs:3-39) before the final order is taken.
#include "px_device.h"
#include "px_kernels.h"
#include "px_scan_common.h"

#include <float.h>

#include <algorithm>

#include <type_traits>

namespace px {

// List capacities: 32 (int ids), 56 and 120 (16-bit offsets, so that 8 and 4 waves fit),
// and 128 (int ids, 2 waves) for the last few k.
int flat_list_capacity(int kl) {
    if (kl <= 32) return 32;
    if (kl <= 56) return 56;
    if (kl <= 120) return 120;
    return 128;
}
bool flat_list_narrow_ids(int kp) { return kp == 32 || kp == 56 || kp == 120; }
// Waves per workgroup: the waves share the corpus stage buffers (two, 67.6 KB of LDS; three
// for lists of 32, 101.4 KB); the per-wave candidate lists take 32 * KP * (4 + id bytes)
// each.
constexpr int flat_waves(int kp) { return kp <= 56 ? 8 : (kp <= 120 ? 4 : 2); }
template <int KP>
struct ListId {
    using type =
        typename std::conditional<KP == 32 || KP == 56 || KP == 120, unsigned short, int>::type;
};
int flat_queries_per_block(int kp) { return 32 * flat_waves(kp); }

// Bulk list fill for the first tile of a split, whose lists start empty: rather
// than inserting the tile's candidates one by one (shifting the list each time), take them
// in ascending (key, row) order, kl rounds of "smallest remaining", so each is appended.
// key[x] is this lane's key of tile row 32 (x / 16) + mfma_row(x % 16, h) for query j;
// lanes l and l ^ 32 hold the two halves of the same query's 64 rows, and within a lane
// rows ascend with x. Rows past the split's end (and padding queries) never qualify.
// Writes slots 0..min(kl, 64)-1 of the query's list (unfilled slots stay (+inf, none))
// and returns its tail (+inf until kl rows qualified).
template <typename IdT>
__device__ __forceinline__ void first_tile_lists(const float (&key)[32], int64_t t0,
                                                 int64_t row1, bool qvalid, int kl, float* lk,
                                                 IdT* li, int base, float& tau_k, int& tau_i) {
    constexpr int kNoKey = 0x7fffffff;  // sorts after every real key's total-order int
    const int h = lane_id() >> 5;
    const int rem = (int)min<int64_t>(row1 - t0, (int64_t)64);
    int tk[32];
#pragma unroll
    for (int x = 0; x < 32; ++x) {
        const int off = (x >> 4) * 32 + mfma_row(x & 15, h);
        tk[x] = (qvalid && off < rem) ? total_key(key[x]) : kNoKey;
    }
    int last_t = kNoKey, last_i = kIdNone;
    for (int r = 0; r < kl; ++r) {
        // this lane's smallest remaining (strict < keeps the lowest row among equal keys)
        int bt = kNoKey, bx = 0;
#pragma unroll
        for (int x = 0; x < 32; ++x) {
            const bool lt = tk[x] < bt;
            bt = lt ? tk[x] : bt;
            bx = lt ? x : bx;
        }
        const int bi = bt == kNoKey ? kIdNone
                                    : (int)(t0 + (bx >> 4) * 32 + mfma_row(bx & 15, h));
        const int pt = __shfl_xor(bt, 32), pi = __shfl_xor(bi, 32);
        const bool mine = bt < pt || (bt == pt && bi < pi);
        const int wt = mine ? bt : pt, wi = mine ? bi : pi;
        if (__ballot(wt != kNoKey) == 0) break;  // fewer than kl rows qualify anywhere
#pragma unroll
        for (int x = 0; x < 32; ++x) tk[x] = (mine && x == bx) ? kNoKey : tk[x];
        if (h == 0 && wt != kNoKey) {
            lk[r] = __int_as_float(wt ^ (int)(((unsigned)(wt >> 31)) >> 1));
            li[r] = id_store<IdT>(wi, base);
        }
        last_t = wt;
        last_i = wi;
        if (r != kl - 1) last_i = kIdNone;
    }
    // the tail is slot kl-1: a real entry only when kl rows qualified
    const bool full = last_i != kIdNone;
    tau_k = full ? __int_as_float(last_t ^ (int)(((unsigned)(last_t >> 31)) >> 1))
                 : __int_as_float(0x7f800000);
    tau_i = full ? last_i : kIdNone;
}

// One workgroup = WAVES waves = 32 * WAVES queries x one corpus split of rows_per_split rows.
//
// MFMA operands: A = corpus rows (M), B = queries (N), K = dims. For the 4 sub-steps e of
// dim group g, lane (i, h) feeds A[i][h] = x[row i][8g + 4h + e] and lane (j, h) feeds
// B[h][j] = q[j][8g + 4h + e]: both sides agree on the dim of every K slot.
//
// Pipeline: the corpus streams through LDS in stages of 64 rows x 128 dims (one tile is
// ceil(dp / 128) stages; MULTI when that is more than one). While the waves run the MFMAs
// of stage s out of one LDS buffer, every thread holds the global loads of stage s + 1 in
// registers and writes them to the other buffer afterwards: one barrier per stage. With
// MULTI each wave's query-chunk registers take the next stage's chunk group by group, as
// the MFMAs release them. Every load is issued in a fixed order on a
// static path, so waiting for one never waits for the prefetch behind it (vector loads
// retire in order). FILT scans the compacted row ids of a filter; the ids of the next
// tile are loaded one stage ahead of the rows themselves.
//
// Selection: each wave keeps, per query, a sorted list of the best kl (key, position)
// candidates of its split in LDS. A candidate must beat the list's last entry (tau) and
// the query's shared threshold gtau, the smallest list tail any split has published so far
// (a valid bound: that split already holds kl rows at or below it), and a second bound
// gbound: every split publishes the key in its list slot m - 1 (m = ceil(kl / P), P =
// min(splits, 32)) to slot (split % 32) of the query's gbest row, so m rows of that split
// sit at or below it; the ceil(kl / m)-th smallest of the published keys (at most P are
// needed) then covers kl rows. gbound is
// recomputed on a geometric schedule of tiles (most of its tightening happens early),
// which cuts list insertions by an order of magnitude over gtau alone. Equal keys pass only
// where they can still matter for the lower-id tie rule: at the shared bound, or when the
// list's tail came from the current tile (earlier tiles hold smaller positions).
//
// COLLECT replaces the lists: each query has a fixed threshold (key, position), and every
// row at or below it is appended, unsorted, to one of two regions of its (query slot,
// split) -- one per lane of the pair that holds the query, each with its own counter, so
// appends need no cross-lane step; flat_collect_select_kernel takes it from there. The
// threshold tests of a tile run during the next tile's MFMAs (both waves of a SIMD reach
// the epilogue together, so an epilogue of its own would leave the matrix unit idle).
template <int KP, int WAVES, bool L2, bool MULTI, bool FILT, bool COLLECT = false, bool H16 = false>
__global__ __launch_bounds__(WAVES * 64) void flat_scan_kernel(FlatScanArgs a) {
    if (a.abort && *a.abort == a.abort_seq) return;
    constexpr int NT = WAVES * 64;
    // H16 (list mode, rows of exactly 128 dims): rows and queries as fp16 (FlatScanArgs::
    // corpus_h, queries_h; every value exact in fp16), 16 dims a MFMA, 256-byte rows in LDS
    // at a 272-byte pitch; else fp32 rows at kLdsStride floats
    constexpr int kRowBytes = H16 ? kChunk * 2 : kChunk * 4;
    constexpr int kPitch = H16 ? kRowBytes + 16 : kLdsStride * 4;
    constexpr int kF4PerRow = kRowBytes / 16;              // 16-byte pieces per staged row
    constexpr int kRowStep = NT / kF4PerRow;               // rows between a thread's loads
    constexpr int kPF = kTileRows / kRowStep;              // pieces per thread per stage
    constexpr int NG = H16 ? 8 : 16;                       // MFMA dim groups per chunk
    static_assert(NT % kF4PerRow == 0 && kTileRows % kRowStep == 0, "uneven stage split");
    static_assert(!H16 || (!MULTI && !COLLECT), "fp16 rows: the one-chunk list scan");
    // Stage buffers and norm slots. Collect mode and lists of 32: three buffers and four
    // norm slots, no barrier per stage (the stage sync of px_collect.hip's scan: a wave may
    // run a stage ahead of the slowest, so that one wave's list insertions or appends do not
    // hold up the others). Longer lists: two buffers (a third does not fit beside them), a
    // barrier per stage.
    constexpr bool RELAXED = COLLECT || KP == 32;
    static_assert(!RELAXED || WAVES == 8, "the stage sync is for eight waves");
    constexpr int kBufs = RELAXED ? 3 : 2, kNorms = RELAXED ? 4 : 2;
    __shared__ __attribute__((aligned(16))) float tile[kBufs][kTileRows * kLdsStride];
    __shared__ __attribute__((aligned(16))) float tnorm[kNorms][kTileRows];
    __shared__ int committed[8];  // RELAXED: the last stage each wave has committed
    __shared__ float lkeys[WAVES][32][KP];
    using IdT = typename ListId<KP>::type;
    __shared__ IdT lids[WAVES][32][KP];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    // Several query chunks (MULTI) over several rounds of workgroups (a.xcd_major): every
    // stage reloads the next chunk of its 256 queries from L2, and every query tile streams
    // the rows of every split. Blocks reach the eight XCDs round-robin by index (block b runs
    // on XCD b % 8), so with the grid padded to a multiple of 8, block b takes position
    // p = (b % 8) * (grid / 8) + b / 8: each XCD works through a contiguous eighth of an
    // order of the (query tile, split) pairs that takes the query tiles in groups of four,
    // a group's splits in turn with its query tiles fastest. The 32 workgroups an XCD holds
    // at once are then about four query tiles x eight splits: their query chunks (1.5 MB)
    // stay in L2 and each row stream serves four of them (10M x 384 with a 10% filter, 16,384
    // queries, HBM fetched a scan: blocks in index order 288 GB at 109.6 ms; a query tile's
    // splits together 77 GB; eight query tiles x four splits 45 GB; four x eight 30 GB, these
    // three within 0.5% of 106.3 ms: HBM is not the bound. One round, 100k x 384 with 1,000
    // queries: 0.771 -> 0.779 ms, so not there).
    int qt = (int)blockIdx.x / a.splits, split = (int)blockIdx.x % a.splits;
    if (MULTI && a.xcd_major) {
        const int qtiles = (a.nq + WAVES * 32 - 1) / (WAVES * 32);
        const int p = (int)(blockIdx.x % 8) * (int)(gridDim.x / 8) + (int)(blockIdx.x / 8);
        if (p >= qtiles * a.splits) return;  // grid padding: before any barrier
        const int grp = p / (4 * a.splits);      // the group of (up to) four query tiles
        const int w = min(4, qtiles - 4 * grp);  // its width: the last may be narrower
        const int rem = p - grp * 4 * a.splits;  // < w splits
        qt = grp * 4 + rem % w;
        split = rem / w;
    }
    const int slot = qt * (WAVES * 32) + wave * 32 + j;
    const bool qvalid = slot < a.nq;
    // collect mode: a wave whose 32 queries are all padding (last query tile) skips its
    // MFMAs and epilogue, so its SIMD is free for the live waves (the list kernel keeps
    // them: its code is tighter without the extra branch, 23.7 against 24.2 ms)
    const bool wave_live = !COLLECT || qt * (WAVES * 32) + wave * 32 < a.nq;
    const int q = (COLLECT && a.qlist) ? a.qlist[qvalid ? slot : 0] : slot;
    const int64_t row0 = (int64_t)split * a.rows_per_split;
    const int64_t row1 = min(a.n_eff, row0 + a.rows_per_split);
    const float kInf = __int_as_float(0x7f800000);
    const int nch = MULTI ? (a.dp + kChunk - 1) / kChunk : 1;
    const int64_t ntiles = (row1 - row0 + kTileRows - 1) / kTileRows;
    const int64_t nstages = ntiles * nch;
    const int cc = tid % kF4PerRow;                        // this thread's float4 column
    const int rr0 = tid / kF4PerRow;                       // its first row in a stage

    if constexpr (!COLLECT) {
        for (int x = lane; x < 32 * KP; x += 64) {
            lkeys[wave][x / KP][x % KP] = kInf;
            lids[wave][x / KP][x % KP] = id_store<IdT>(kIdNone, 0);
        }
    }
    float tau_k = kInf;   // this wave's list tail for query j (slot kl-1)
    int tau_i = kIdNone;
    int published = 0x7fffffff;
    // published list slot pub_m - 1, so that pub_rank <= min(splits, 32) publishers cover kl
    const int pub_m = (a.kl + min(a.splits, 32) - 1) / min(a.splits, 32);
    const int pub_rank = (a.kl + pub_m - 1) / pub_m;
    int published_best = kTotalKeyInf;
    float gbound = kInf;
    int64_t next_refresh = 1;                                // tile index of the next refresh
    const float* qrow = a.queries + (int64_t)(qvalid ? q : 0) * a.dp;
    int* gtau = COLLECT ? nullptr : a.gtau + (qvalid ? q : 0);
    // collect mode with a.gbest: a shared bound as well (below)
    int* gbest = (COLLECT && !a.gbest) ? nullptr : a.gbest + (qvalid ? q : 0);
    // collect mode: this query's threshold (nothing passes -inf) and region
    float cthr = -kInf;
    int cpos = -1, ccount = 0;
    // Collect mode's shared bound (a.gbest set, a.kl <= min(splits, 32)): each lane
    // publishes the smallest key of its rows of the split so far to the query's slot
    // split % 32 (atomicMin; the two lanes of a pair share the slot), so every published
    // slot has a row of its own splits at or below it, and the kl-th smallest slot bounds
    // the query's best kl. A row passes when it is at or below both the threshold and
    // gbound; ctest = min(cthr, gbound) pre-screens a tile's keys.
    // The first tile of a split also bounds itself: its kl-th smallest key has kl of the
    // split's rows at or below it (so a query needs no threshold), and the first refresh
    // comes right after the first tile's publication.
    // (one query chunk and no filter only: the host applies it to unfiltered searches of
    // rows of at most 128 padded dims)
    const bool dyn = COLLECT && !MULTI && !FILT && a.gbest != nullptr && !a.dense;
    int cpub = kTotalKeyInf;
    bool pub_now = false;  // publish cpub after this stage's commit
    float ctest = -kInf;
    if (dyn) next_refresh = 0;
    // list mode with one query chunk: the insertions of a tile's second row block run during
    // the next tile's MFMAs (an insertion otherwise holds up the stage barrier for all eight
    // waves); the first block's run in the epilogue, as do all of them with MULTI, and with a
    // filter on L2 rows, where the 16 deferred keys pushed 3-4 registers to scratch
    // (1M x 128, 10,000 queries, k = 10, without the deferral: 10% filter 3.39 -> 3.28 ms,
    // 50% filter 12.87 -> 13.05)
    constexpr bool LDEFER = !COLLECT && !MULTI && !(FILT && L2);
    float pkey[COLLECT ? 32 : (LDEFER ? 16 : 1)];  // keys of the previous tile tested during this one
    float pthr = -kInf;            // list mode: the previous tile's threshold (as thr2 below)
    int pt0 = 0, prem = 0;         // its first position and (collect mode) row count
    bool pend = false;             // some lane of the wave has a key at or below its threshold
    auto collect_x = [&](int x) {
        if constexpr (COLLECT) {
            const int off = (x >> 4) * 32 + mfma_row(x & 15, h);
            const float kv = pkey[x];
            const bool p = off < prem && (kv < cthr || (kv == cthr && pt0 + off <= cpos)) &&
                           kv <= gbound;
            if (p) {
                PX_DCHECK(a.dbg, kDbgFlat, qvalid && pt0 + off < a.n_eff);
                if (ccount < a.cap) {
                    const int64_t at =
                        (((int64_t)slot * a.splits + split) * 2 + h) * a.cap + ccount;
                    a.cand_keys[at] = kv;
                    a.cand_pos[at] = pt0 + off;
                }
                ++ccount;
            }
        }
    };
    // list mode: the candidates of row x (16..31) of the previous tile, one insertion at a
    // time in lane order, each checked against the current tail of its query's list
    auto list_x = [&](int x) {
        if constexpr (LDEFER) {
            const int r = x & 15;
            unsigned long long m = __ballot(pkey[r] <= pthr);
            while (m) {
                const int src = __builtin_ctzll(m);
                m &= m - 1;
                const float ck = readlane_f(pkey[r], src);
                const int cid = pt0 + 32 + mfma_row(r, src >> 5);
                const float tk = readlane_f(tau_k, src);
                const int ti = readlane_i(tau_i, src);
                if (!cand_less(ck, cid, tk, ti)) continue;
                const int ql = src & 31;
                float nk;
                int ni;
                list_insert<KP>(&lkeys[wave][ql][0], &lids[wave][ql][0], (int)row0, a.kl, ck,
                                cid, nk, ni);
                if (j == ql) {
                    tau_k = nk;
                    tau_i = ni;
                }
            }
        }
    };
    // list mode: publish a tightened list tail as the query's shared bound, and the key in
    // list slot pub_m - 1 to the query's gbest slot of this split. atomicMin, not a plain
    // store: a plain store would stay in this XCD's L2, out of sight of the splits running
    // on the other XCDs.
    auto publish = [&]() {
        if constexpr (!COLLECT) {
            const int tk = total_key(tau_k);
            if (h == 0 && qvalid && tau_i != kIdNone && tk < published) {
                atomicMin(gtau, tk);
                published = tk;
            }
            const int bk = total_key(lkeys[wave][j][pub_m - 1]);
            if (h == 0 && qvalid && bk < published_best) {
                atomicMin(gbest + (int64_t)(split & 31) * a.gbest_ld, bk);
                published_best = bk;
            }
        }
    };
    if constexpr (COLLECT) {
        if (qvalid && !a.dense) {
            cthr = from_total_key(a.thr_key[q]);
            cpos = a.thr_pos[q];
        }
    }

    // Every load below is unconditional (clamped to a valid address) so that the number of
    // loads in flight is known statically; values are zeroed where they are consumed, not
    // where they are loaded, so that no select waits for a load.
    auto zero_unless = [](bool keep, float4 v) {
        v.x = keep ? v.x : 0.f;
        v.y = keep ? v.y : 0.f;
        v.z = keep ? v.z : 0.f;
        v.w = keep ? v.w : 0.f;
        return v;
    };
    // raw query chunk c (dims past the chunk's end are loaded clamped, zeroed by b_valid)
    auto load_b = [&](int c, float4 (&bb)[16]) {
        const int dc = min(kChunk, a.dp - c * kChunk);
#pragma unroll
        for (int g = 0; g < 16; ++g)
            bb[g] = *reinterpret_cast<const float4*>(qrow + c * kChunk + min(g * 8 + h * 4, dc - 4));
    };
    auto b_valid = [&](int c, int g) {
        return qvalid && g * 8 + h * 4 < min(kChunk, a.dp - c * kChunk);
    };
    // Row ids (-1 past the split's end) of the rows this thread stages for tile t, and of
    // row t0 + tid whose norm it stages.
    int rid[kPF], pid;
    auto tile_ids = [&](int64_t t) {
        const int64_t t0 = row0 + t * kTileRows;
#pragma unroll
        for (int u = 0; u < kPF; ++u) {
            const int64_t pos = t0 + rr0 + u * kRowStep;
            const int v = FILT ? a.rowidx[min(pos, row1 - 1)] : (int)pos;
            rid[u] = pos < row1 ? v : -1;
            PX_DCHECK(a.dbg, kDbgFlat, pos >= row1 || (v >= 0 && v < a.rows));
        }
        const int64_t pos = t0 + tid;
        const int v = FILT ? a.rowidx[min(pos, row1 - 1)] : (int)pos;
        pid = (tid < kTileRows && pos < row1) ? v : -1;
    };
    float4 pf[kPF];
    float pn = 0.f;
    unsigned pvalid = 0;  // bit u: pf[u] is a real row's data; bit kPF: pn is a real norm
    // (stages are addressed by chunk c and tile parity, kept incrementally: a 64-bit division
    // of the stage index by the chunk count costs dozens of scalar instructions a stage)
    auto fetch = [&](int c) {
        const int f4r = min(kChunk, a.dp - c * kChunk) >> 2;
        pvalid = 0;
#pragma unroll
        for (int u = 0; u < kPF; ++u) {
            if constexpr (H16) {
                pf[u] = *reinterpret_cast<const float4*>(a.corpus_h + (int64_t)max(rid[u], 0) * kChunk +
                                                         cc * 8);
                pvalid |= rid[u] >= 0 ? 1u << u : 0u;
            } else {
                pf[u] = *reinterpret_cast<const float4*>(
                    a.corpus + (int64_t)max(rid[u], 0) * a.dp + c * kChunk + min(cc, f4r - 1) * 4);
                pvalid |= (rid[u] >= 0 && cc < f4r) ? 1u << u : 0u;
            }
        }
        if (L2) {
            pn = a.norms[max(pid, 0)];
            pvalid |= pid >= 0 ? 1u << kPF : 0u;
        }
    };
    // stage buffer sb, chunk c, tile parity tp
    auto commit = [&](int sb, int c, int tp) {
        char* tb = reinterpret_cast<char*>(tile[sb]);
#pragma unroll
        for (int u = 0; u < kPF; ++u)
            *reinterpret_cast<float4*>(tb + (rr0 + u * kRowStep) * kPitch + cc * 16) =
                zero_unless((pvalid >> u) & 1u, pf[u]);
        if (L2 && c == 0 && tid < kTileRows)
            tnorm[tp][tid] = (pvalid >> kPF) & 1u ? pn : 0.f;
    };
    // chunk and tile of the stage after one of chunk c and tile t
    auto next_stage = [&](int c, int64_t t, int& cn, int64_t& tn) {
        cn = c + 1 == nch ? 0 : c + 1;
        tn = cn == 0 ? t + 1 : t;
    };

    // B operands: query chunk 0 (H16: dims 16 g + 8 h .. + 7 in fp16; zero for padding slots)
    using Frag = std::conditional_t<H16, f16x8, float4>;
    Frag b[NG];
    if constexpr (H16) {
        const unsigned short* qh = a.queries_h + (int64_t)(qvalid ? q : 0) * kChunk + h * 8;
#pragma unroll
        for (int g = 0; g < NG; ++g)
            b[g] = qvalid ? *reinterpret_cast<const f16x8*>(qh + g * 16) : f16x8{};
    } else {
        load_b(0, b);
#pragma unroll
        for (int g = 0; g < 16; ++g) b[g] = zero_unless(b_valid(0, g), b[g]);
    }
    if (nstages > 0) {
        tile_ids(0);
        fetch(0);
        commit(0, 0, 0);
        if constexpr (RELAXED) {
            // stage 1 in LDS too, ids for the tile of stage 2
            int c1, c2;
            int64_t t1, t2;
            next_stage(0, 0, c1, t1);
            next_stage(c1, t1, c2, t2);
            tile_ids(t1);
            fetch(c1);
            commit(1, c1, (int)(t1 & (kNorms - 1)));
            tile_ids(t2);
        } else {
            tile_ids(nch > 1 ? 0 : 1);  // ids for the tile of stage 1
        }
    }
    if (RELAXED && tid < 8) committed[tid] = 1;
    __syncthreads();
    const unsigned caddr = (unsigned)(uintptr_t)(committed + (lane & 7));

    if constexpr (!COLLECT) {
        // A wave whose 32 queries are all padding (small batches) only helps stage the
        // corpus: same loads, same barriers, no MFMAs, no selection. A separate loop, so
        // that the live waves' code is the one the full batches run.
        if (qt * (WAVES * 32) + wave * 32 >= a.nq) {
            int c = 0;
            int64_t t = 0;
            int rb = 0;
            for (int64_t s = 0; s < nstages; ++s) {
                int c1, c2;
                int64_t t1, t2;
                next_stage(c, t, c1, t1);
                next_stage(c1, t1, c2, t2);
                if constexpr (RELAXED) {
                    int c3;
                    int64_t t3;
                    next_stage(c2, t2, c3, t3);
                    fetch(c2);
                    tile_ids(t3);
                    if (stage_wait(caddr, (int)(s + 1), a.spin_limit) >= a.spin_limit &&
                        a.spin_fail && lane == 0)
                        atomicOr(a.spin_fail, 1);
                    commit(rb == 0 ? 2 : rb - 1, c2, (int)(t2 & (kNorms - 1)));
                    stage_publish(committed, wave, lane, (int)(s + 2));
                    rb = rb == 2 ? 0 : rb + 1;
                } else {
                    fetch(c1);
                    tile_ids(t2);
                    commit((int)((s + 1) & 1), c1, (int)(t1 & 1));
                    __syncthreads();
                }
                c = c1;
                t = t1;
            }
            return;
        }
    }

    f32x16 acc0 = {0.f}, acc1 = {0.f};
    int c = 0;        // chunk of stage s
    int64_t ti = 0;   // its tile
    int rb = 0;       // RELAXED: its stage buffer (s % 3)
    for (int64_t s = 0; s < nstages; ++s) {
        int c1, c2, c3 = 0;
        int64_t t1, t2, t3 = 0;
        next_stage(c, ti, c1, t1);
        next_stage(c1, t1, c2, t2);
        if constexpr (RELAXED) next_stage(c2, t2, c3, t3);
        const int64_t t0 = row0 + ti * kTileRows;
        // the shared bound, loaded in the stage whose epilogue reads it (a tile's last chunk):
        // with several chunks the other stages' loads would go unused (100k x 384, 1,000
        // queries: 0.767 -> 0.762 ms a scan)
        int gt_raw = kTotalKeyInf;
        if constexpr (!COLLECT) {
            if (c == nch - 1)
                gt_raw = __hip_atomic_load(gtau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // MULTI: each b[g] takes the next stage's query chunk as soon as this stage's MFMAs
        // have read it. Those loads are not zeroed past the chunk's end or for padding
        // queries: the corpus tile is zero in columns past the chunk's end, every value is
        // finite, and padding queries' keys are never used.
        const int cn = c1;
        const int dcn = min(kChunk, a.dp - cn * kChunk);
        // barrier per stage: stage s + 1's loads and the ids of stage s + 2's tile; RELAXED:
        // stage s + 2's and stage s + 3's (past the last stage every row is -1: harmless
        // clamped loads)
        if constexpr (RELAXED) {
            fetch(c2);
            tile_ids(t3);
        } else {
            fetch(c1);
            tile_ids(t2);
        }
        if (c == 0) {
            acc0 = (f32x16){0.f};
            acc1 = (f32x16){0.f};
        }
        const int ng = !wave_live ? 0 : H16 ? NG : min(kChunk, a.dp - c * kChunk) >> 3;
        const int sb = RELAXED ? rb : (int)(s & 1);
        // rows j and 32 + j, the lane's 16 bytes of each 32-byte dim group
        const char* ta0 = reinterpret_cast<const char*>(tile[sb]) + j * kPitch + h * 16;
        const char* ta1 = ta0 + 32 * kPitch;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            if (g < ng) {
                const Frag a0 = *reinterpret_cast<const Frag*>(ta0 + g * 32);
                const Frag a1 = *reinterpret_cast<const Frag*>(ta1 + g * 32);
                acc0 = mfma_group(a0, b[g], acc0);
                acc1 = mfma_group(a1, b[g], acc1);
            }
            if constexpr (MULTI)
                b[g] = *reinterpret_cast<const float4*>(qrow + cn * kChunk +
                                                        min(g * 8 + h * 4, dcn - 4));
            if constexpr (COLLECT) {
                // one compare per row and one uniform branch per pair of rows; the exact
                // test and the append only where some lane has a row at or below
                if (pend && __ballot(pkey[2 * g] <= ctest || pkey[2 * g + 1] <= ctest)) {
                    collect_x(2 * g);
                    collect_x(2 * g + 1);
                }
            }
            if constexpr (LDEFER) {
                // the previous tile's rows 16 .. 31, one (H16: two) a group
                if (pend) {
                    list_x(16 + (16 / NG) * g);
                    if constexpr (H16) list_x(17 + 2 * g);
                }
            }
        }
        if constexpr (COLLECT) pend = false;
        if constexpr (LDEFER) {
            if (pend) {
                publish();
                pend = false;
            }
        }

        // The tile epilogue (keys, tests, list insertions). Lists of 32 and collect mode run it
        // after their commit of stage s + 2, so that one wave's tests and insertions hold up no
        // other wave's next stage (100k x 384 lists: 0.709 -> 0.702 ms on the resident-query
        // kernel; 1M x 128 lists, 1,000 queries: 2.325 -> 2.313 ms); with a barrier per stage
        // it runs before the commit, as the barrier waits for it either way.
        auto tile_epilogue = [&]() __attribute__((always_inline)) {
            if (c == nch - 1 && wave_live) {
                // Epilogue, branch-free: keys of the 32 rows this lane holds for query j.
                // L2 drops the per-query constant ||q||^2 (it does not change a query's order;
                // the merge re-ranks exactly), so key = ||x||^2 - 2 q.x; IP key = -q.x.
                // (collect mode writes them straight into pkey, where the next tile's MFMA loop
                // tests them: the previous tile's keys there have been tested already)
                const float* tn = tnorm[ti & (kNorms - 1)];
                float key_own[COLLECT ? 1 : 32];
                auto& key = [&]() -> float(&)[32] {
                    if constexpr (COLLECT) return pkey;
                    else return key_own;
                }();
                float kmin = kInf;
    #pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
    #pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
                        const int lr = rb * 32 + 8 * r4 + 4 * h;  // rows lr .. lr+3
                        float4 nv = make_float4(0.f, 0.f, 0.f, 0.f);
                        if (L2) nv = *reinterpret_cast<const float4*>(tn + lr);
                        const float nn[4] = {nv.x, nv.y, nv.z, nv.w};
    #pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * r4 + e;
                            const float dot = rb == 0 ? acc0[r] : acc1[r];
                            const float kv = L2 ? __builtin_fmaf(-2.0f, dot, nn[e]) : -dot;
                            key[rb * 16 + r] = kv;
                            kmin = fminf(kmin, kv);
                        }
                    }
                }
                if constexpr (COLLECT) {
                    const int rem = (int)min<int64_t>(row1 - t0, (int64_t)kTileRows);
                    if (a.dense) {
                        // every key of the tile, row-major by position (+inf past the split's
                        // end), so that each query's keys are contiguous for the ladder: keys
                        // 4 m .. 4 m + 3 of this lane are four consecutive rows
                        if (qvalid) {
                            float* dst = a.cand_keys + (int64_t)slot * a.dense_ld + t0;
    #pragma unroll
                            for (int m = 0; m < 8; ++m) {
                                float v[4];
    #pragma unroll
                                for (int e = 0; e < 4; ++e) {
                                    const int x = 4 * m + e;
                                    v[e] = (x >> 4) * 32 + mfma_row(x & 15, h) < rem ? key[x] : kInf;
                                }
                                const int lr = (m >> 2) * 32 + 8 * (m & 3) + 4 * h;
                                *reinterpret_cast<float4*>(dst + lr) = make_float4(v[0], v[1], v[2], v[3]);
                            }
                        }
                    } else {
                    // tested during the next tile's MFMAs (or after the last tile); with MULTI
                    // (several chunks per tile, and the next query chunk held in registers) the
                    // keys are tested here instead, so that they are not held across the MFMAs
                    if (dyn) {
                        // this lane's smallest key of the split's rows so far (the last tile
                        // of a split may end early: rows past its end do not count)
                        float vmin = kmin;
                        if (rem < kTileRows) {
                            vmin = kInf;
    #pragma unroll
                            for (int x = 0; x < 32; ++x)
                                vmin = (x >> 4) * 32 + mfma_row(x & 15, h) < rem ? fminf(vmin, key[x])
                                                                                 : vmin;
                        }
                        // (only where some query of the wave has no threshold: a sampled one
                        // already bounds the first tile far below its k'-th key)
                        if (t0 == row0 && __ballot(qvalid && cthr == kInf))
                            gbound = first_tile_kth(key, rem, qvalid, a.kl);
                        // published after the stage's commit: its waits then do not wait for the
                        // atomic, which has the next tile's MFMAs to complete
                        const int tk = total_key(vmin);
                        pub_now = qvalid && tk < cpub;
                        cpub = pub_now ? tk : cpub;
                        if (ti == next_refresh) {
                            int v[16];
                            load_slots16(gbest, a.gbest_ld, h, v);
                            gbound = fminf(gbound, from_total_key(kth_smallest32(v, a.kl)));
                            // sparser than the lists' schedule: each refresh waits for its loads
                            // in the epilogue (t -> t + t/4: 21.73 ms a scan on 1M x 128, t + t/2:
                            // 21.58, t -> 2t: 21.58)
                            next_refresh = ti + max<int64_t>(1, ti >> 1);
                        }
                    }
                    ctest = fminf(cthr, gbound);
                    pt0 = (int)t0;
                    prem = rem;
                    pend = __ballot(kmin <= ctest) != 0;
                    if constexpr (MULTI) {
                        if (pend) {
    #pragma unroll
                            for (int g = 0; g < 16; ++g) {
                                if (__ballot(pkey[2 * g] <= ctest || pkey[2 * g + 1] <= ctest)) {
                                    collect_x(2 * g);
                                    collect_x(2 * g + 1);
                                }
                            }
                        }
                        pend = false;
                    }
                    }
                } else {
                // Padding queries get a threshold nothing passes; rows past the split's end
                // (last tile only) compare as NaN below.
                if (ti == next_refresh) {
                    // loaded here rather than ahead: refreshes are rare, and holding 16 more
                    // registers across the MFMAs would spill
                    int v[16];
                    load_slots16(gbest, a.gbest_ld, h, v);
                    gbound = fminf(gbound, from_total_key(kth_smallest32(v, pub_rank)));
                    // t -> t + t/2: each refresh stalls both waves of a SIMD for its loads (on
                    // 100k x 384 x 1,000 queries, 25 tiles a split: 0.81 -> 0.80 ms against
                    // t + t/4; t -> 2t loses 1% on 1M x 128 and on 128 queries at k = 100)
                    next_refresh = ti + max<int64_t>(1, ti >> 1);
                }
                const float thr =
                    qvalid ? fminf(fminf(tau_k, from_total_key(gt_raw)), gbound) : -kInf;
                if (t0 == row0) {
                    // First tile of the split: the lists are empty, so instead of inserting the
                    // tile's candidates one by one, sort them. Each lane sorts its 32 (key, row)
                    // pairs, merges them with its partner lane's (same query, other 32 rows)
                    // and the pair writes the query's best kl as its list.
                    first_tile_lists(key, t0, row1, qvalid, a.kl, &lkeys[wave][j][0],
                                     &lids[wave][j][0], (int)row0, tau_k, tau_i);
                    publish();
                } else {
                    const int rem = (int)min<int64_t>(row1 - t0, (int64_t)kTileRows);
                    const bool eq_ok = thr < tau_k || tau_i >= t0;
                    // rows of the first block now (all of them without LDEFER)
                    constexpr int XN = LDEFER ? 16 : 32;
                    // one compare a row: key <= thr2 is key < thr, or key == thr where equal
                    // keys may still enter; rows past the split's end (its last tile) are NaN,
                    // which no compare passes and fminf skips (the test took 17 instructions and
                    // two branches a row with the tie rule and the row bound in it)
                    const float thr2 = eq_ok ? thr : next_below(thr);
                    if (rem < kTileRows) {
    #pragma unroll
                        for (int x = 0; x < 32; ++x)
                            key[x] = (x >> 4) * 32 + mfma_row(x & 15, h) < rem
                                         ? key[x] : __int_as_float(0x7fc00000);
                    }
                    float kmin0 = kInf;
    #pragma unroll
                    for (int x = 0; x < XN; ++x) kmin0 = fminf(kmin0, key[x]);
                    if (__ballot(kmin0 <= thr2)) {
    #pragma unroll
                        for (int x = 0; x < XN; ++x) {
                            const int rb = x >> 4, r = x & 15;
                            unsigned long long m = __ballot(key[x] <= thr2);
                            while (m) {
                                const int src = __builtin_ctzll(m);
                                m &= m - 1;
                                const float ck = readlane_f(key[x], src);
                                const int cid = (int)(t0 + rb * 32 + mfma_row(r, src >> 5));
                                const float tk = readlane_f(tau_k, src);
                                const int ti = readlane_i(tau_i, src);
                                if (!cand_less(ck, cid, tk, ti)) continue;
                                const int ql = src & 31;
                                float nk;
                                int ni;
                                list_insert<KP>(&lkeys[wave][ql][0], &lids[wave][ql][0], (int)row0,
                                                a.kl, ck, cid, nk, ni);
                                if (j == ql) {
                                    tau_k = nk;
                                    tau_i = ni;
                                }
                            }
                        }
                        publish();
                    }
                    if constexpr (LDEFER) {
                        // the second block: during the next tile's MFMAs (or after the last)
                        float kmin1 = kInf;
    #pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            pkey[r] = key[16 + r];
                            kmin1 = fminf(kmin1, key[16 + r]);
                        }
                        pt0 = (int)t0;
                        pthr = thr2;
                        pend = __ballot(kmin1 <= thr2) != 0;
                    }
                }
                }  // !COLLECT
            }
        };
        if constexpr (!RELAXED) tile_epilogue();
        if constexpr (RELAXED) {
            // every wave has committed stage s + 1 (so none still reads stage s - 1, whose
            // buffer and norm slot stage s + 2 takes), then this wave's part of stage s + 2
            if (stage_wait(caddr, (int)(s + 1), a.spin_limit) >= a.spin_limit && a.spin_fail &&
                lane == 0)
                atomicOr(a.spin_fail, 1);
            pair_priority(__hip_atomic_load(committed + (wave ^ 4), __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_WORKGROUP),
                          (int)(s + 1));
            commit(rb == 0 ? 2 : rb - 1, c2, (int)(t2 & (kNorms - 1)));
            stage_publish(committed, wave, lane, (int)(s + 2));
        } else {
            commit((int)((s + 1) & 1), c1, (int)(t1 & 1));
        }
        if constexpr (RELAXED) tile_epilogue();
        if (dyn && pub_now) {
            atomicMin(gbest + (int64_t)(split & 31) * a.gbest_ld, cpub);
            pub_now = false;
        }
        if constexpr (!RELAXED) __syncthreads();
        rb = rb == 2 ? 0 : rb + 1;
        c = c1;
        ti = t1;
    }

    if constexpr (COLLECT) {
        if (pend) {
#pragma unroll
            for (int x = 0; x < 32; ++x) collect_x(x);
        }
        if (qvalid && !a.dense) a.cand_count[((int64_t)slot * a.splits + split) * 2 + h] = ccount;
        return;
    }
    if constexpr (LDEFER) {
        if (pend) {
#pragma unroll
            for (int x = 16; x < 32; ++x) list_x(x);
        }
    }
    // Write this split's lists: part[q][split][0..kl)
    const int qbase = qt * (WAVES * 32) + wave * 32;
    for (int ql = 0; ql < 32; ++ql) {
        const int qq = qbase + ql;
        if (qq >= a.nq) break;
        float* pk = a.part_keys + ((int64_t)qq * a.splits + split) * a.kl;
        int* pi = a.part_ids + ((int64_t)qq * a.splits + split) * a.kl;
        for (int s = lane; s < a.kl; s += 64) {
            pk[s] = lkeys[wave][ql][s];
            pi[s] = id_load(lids[wave][ql][s], (int)row0);
            PX_DCHECK(a.dbg, kDbgFlat, pi[s] == kIdNone || (pi[s] >= row0 && pi[s] < row1));
        }
    }
}

template <int KP, int WAVES, bool L2, bool MULTI, bool H16 = false>
static void launch_scan_f(const FlatScanArgs& a, dim3 grid, hipStream_t s) {
    if (a.rowidx)
        hipLaunchKernelGGL((flat_scan_kernel<KP, WAVES, L2, MULTI, true, false, H16>), grid,
                           dim3(WAVES * 64), 0, s, a);
    else
        hipLaunchKernelGGL((flat_scan_kernel<KP, WAVES, L2, MULTI, false, false, H16>), grid,
                           dim3(WAVES * 64), 0, s, a);
}

template <int KP, int WAVES>
static hipError_t launch_scan_t(const FlatScanArgs& a, hipStream_t s) {
    const int qpb = 32 * WAVES;
    const int64_t qtiles = (a.nq + qpb - 1) / qpb;
    const bool multi = a.dp > kChunk;
    // several chunks: the grid is padded to a multiple of the 8 XCDs (see flat_scan_kernel)
    const bool xm = multi && a.xcd_major;
    const dim3 grid((unsigned)(xm ? (qtiles * a.splits + 7) / 8 * 8 : qtiles * a.splits));
    // fp16 rows and queries (both or neither): rows of exactly 128 dims
    if ((a.corpus_h == nullptr) != (a.queries_h == nullptr) || (a.corpus_h && a.dp != kChunk))
        return hipErrorInvalidValue;
    if (a.corpus_h) {
        if (a.metric == 0) launch_scan_f<KP, WAVES, true, false, true>(a, grid, s);
        else launch_scan_f<KP, WAVES, false, false, true>(a, grid, s);
    } else if (a.metric == 0) {
        if (multi) launch_scan_f<KP, WAVES, true, true>(a, grid, s);
        else launch_scan_f<KP, WAVES, true, false>(a, grid, s);
    } else {
        if (multi) launch_scan_f<KP, WAVES, false, true>(a, grid, s);
        else launch_scan_f<KP, WAVES, false, false>(a, grid, s);
    }
    return hipGetLastError();
}

// Lists of 32 over rows of 129-384 padded dims (list_resident_queries), and the collect scan
// of such rows (COLLECT): 8 waves x 16 queries a workgroup on v_mfma_f32_16x16x4f32, each
// wave holding all of its queries' dims in registers (24-96 VGPRs), so no stage reloads a
// query chunk (flat_scan_kernel's multi-chunk scans reload each lane's next 128 dims every
// stage: 16 loads and their address arithmetic).
// Per stage (64 rows x 128 dims) a wave multiplies 4 row blocks of 16 rows by 8 groups of 16
// dims, 4 MFMAs a group and block, the 4 blocks' accumulators interleaved. MFMA operands:
// lane l = (i, d) with i = l % 16, d = l / 16; in group u, sub-step e, lane l feeds
// A[i][d] = x[row 16 b + i][16 u + 4 d + e] and B[d][j] = q[j = l % 16][16 u + 4 d + e], so
// both sides agree on the dim of every K slot and each lane reads 16 contiguous bytes a
// group (b128 LDS reads; the 132-float pitch keeps them conflict-free); the result holds
// D[4 d + r][j] in register r, so lane l has the keys of query l % 16 for rows
// 16 b + 4 d + r, and the four lanes l % 16 + 16 d share a query.
// The queries are held scaled by the key's factor (-2 for L2, -1 for IP; a power of two, so
// products and sums round as the unscaled ones do, products in the subnormal range aside):
// the accumulators end as -2 q.x or -q.x, and a key is one add of ||x||^2 (the single
// rounding of fma(-2, q.x, ||x||^2)) or the accumulator itself; these keys only choose the
// candidates the merge or the select re-ranks exactly. FULL (dp = NCH x 128): every dim
// group is real and the group loop runs unguarded, so the compiler can keep LDS reads in
// flight ahead of the MFMAs (1.4% on 100k x 384).
// Staging, stage sync, the shared bounds and the list insertions are flat_scan_kernel's
// (lists of 32, three stage buffers, no barrier per stage), with two differences: a wave
// commits its part of stage s + 2 before its tile epilogue rather than after it, so that its
// insertions hold up no other wave (100k x 384, 1,000 queries: 0.709 -> 0.702 ms), and the
// waves of a SIMD keep one issue priority (pair_priority measured 0.3% slower here). The
// split's first tile fills the lists by ordered extraction over the query's four lanes.
// COLLECT (not the dense threshold-sample scans, which stay on flat_scan_kernel): per query a
// threshold (key, position) and two regions a split, as flat_scan_kernel's collect mode lays
// them out; region d / 2 is shared by the lanes d = 0, 1 (and 2, 3), which append a key
// index's rows in lane order, each keeping the region's count.
template <bool L2, bool FILT, int NCH, bool FULL, bool COLLECT>
__global__ __launch_bounds__(512) void flat_list16q_kernel(FlatScanArgs a) {
    if (a.abort && *a.abort == a.abort_seq) return;
    constexpr int WAVES = 8, NT = 512, KP = 32, QW = 16;
    constexpr int kF4PerRow = kChunk / 4, kRowStep = NT / kF4PerRow, kPF = kTileRows / kRowStep;
    constexpr int kBufs = 3, kNorms = 4;
    static_assert(NCH >= 2 && NCH <= 3, "rows of 129-384 padded dims");
    __shared__ __attribute__((aligned(16))) float tile[kBufs][kTileRows * kLdsStride];
    __shared__ __attribute__((aligned(16))) float tnorm[kNorms][kTileRows];
    __shared__ int committed[8];
    __shared__ float lkeys[COLLECT ? 1 : WAVES][QW][KP];
    __shared__ unsigned short lids[COLLECT ? 1 : WAVES][QW][KP];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, j = lane & 15, d = (lane >> 4) & 3, h = lane >> 5;
    int qt = (int)blockIdx.x / a.splits, split = (int)blockIdx.x % a.splits;
    if (a.xcd_major) {
        // flat_scan_kernel's XCD-major order of (query tile, split) pairs, in groups of 16
        // query tiles: with the queries in registers, an XCD's L2 holds only row streams, so
        // about 16 query tiles x 2 splits at once share each (10M x 384 with a 10% filter,
        // 16,384 queries, HBM fetched a collect scan: groups of 4 56 GB, of 16 12.5 GB)
        const int qtiles = (a.nq + WAVES * QW - 1) / (WAVES * QW);
        const int p = (int)(blockIdx.x % 8) * (int)(gridDim.x / 8) + (int)(blockIdx.x / 8);
        if (p >= qtiles * a.splits) return;  // grid padding: before any barrier
        const int grp = p / (16 * a.splits), w = min(16, qtiles - 16 * grp);
        const int rem = p - grp * 16 * a.splits;
        qt = grp * 16 + rem % w;
        split = rem / w;
    }
    const int slot = qt * (WAVES * QW) + wave * QW + j;
    const bool qvalid = slot < a.nq;
    const int q = (COLLECT && a.qlist) ? a.qlist[qvalid ? slot : 0] : slot;
    const int64_t row0 = (int64_t)split * a.rows_per_split;
    const int64_t row1 = min(a.n_eff, row0 + a.rows_per_split);
    const float kInf = __int_as_float(0x7f800000);
    const int64_t ntiles = (row1 - row0 + kTileRows - 1) / kTileRows;
    const int64_t nstages = ntiles * NCH;
    const int cc = tid % kF4PerRow, rr0 = tid / kF4PerRow;

    if constexpr (!COLLECT) {
        for (int x = lane; x < QW * KP; x += 64) {
            lkeys[wave][x / KP][x % KP] = kInf;
            lids[wave][x / KP][x % KP] = 0xffff;
        }
    }
    float tau_k = kInf;  // the list tail of query j (slot kl - 1), in all four of its lanes
    int tau_i = kIdNone;
    int published = 0x7fffffff;
    const int pub_m = (a.kl + min(a.splits, 32) - 1) / min(a.splits, 32);
    const int pub_rank = (a.kl + pub_m - 1) / pub_m;
    int published_best = kTotalKeyInf;
    float gbound = kInf;
    int64_t next_refresh = 1;
    int* gtau = COLLECT ? nullptr : a.gtau + (qvalid ? q : 0);
    int* gbest = COLLECT ? nullptr : a.gbest + (qvalid ? q : 0);
    // collect mode: the query's threshold (key, position; nothing passes -inf) and the count
    // of its region of this split: region h = d / 2, shared by lanes d = 2 h and 2 h + 1
    // (rows 16 b + 8 h .. + 7 of each block: at most half the split's rows), the even lane's
    // rows of a key index x first; both lanes keep the same count
    float cthr = -kInf;
    int cpos = -1, ccount = 0;
    if constexpr (COLLECT) {
        if (qvalid) {
            cthr = from_total_key(a.thr_key[q]);
            cpos = a.thr_pos[q];
        }
    }
    auto publish = [&]() {
        const int tk = total_key(tau_k);
        if (d == 0 && qvalid && tau_i != kIdNone && tk < published) {
            atomicMin(gtau, tk);
            published = tk;
        }
        const int bk = total_key(lkeys[wave][j][pub_m - 1]);
        if (d == 0 && qvalid && bk < published_best) {
            atomicMin(gbest + (int64_t)(split & 31) * a.gbest_ld, bk);
            published_best = bk;
        }
    };

    // the queries (B operands) times the key's factor, held for the whole scan: chunk c,
    // group u: dims c 128 + 16 u + 4 d .. + 3 (whole float4s inside or past dp, dp being a
    // multiple of 8)
    float4 bq[NCH][8];
    {
        const float* qrow = a.queries + (int64_t)(qvalid ? q : 0) * a.dp;
        const float f = L2 ? -2.0f : -1.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int dim = c * kChunk + 16 * u + 4 * d;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (qvalid && dim < a.dp) v = *reinterpret_cast<const float4*>(qrow + dim);
                bq[c][u] = make_float4(f * v.x, f * v.y, f * v.z, f * v.w);
            }
    }

    auto zero_unless = [](bool keep, float4 v) {
        v.x = keep ? v.x : 0.f;
        v.y = keep ? v.y : 0.f;
        v.z = keep ? v.z : 0.f;
        v.w = keep ? v.w : 0.f;
        return v;
    };
    int rid[kPF], pid;
    auto tile_ids = [&](int64_t t) {
        const int64_t t0 = row0 + t * kTileRows;
#pragma unroll
        for (int u = 0; u < kPF; ++u) {
            const int64_t pos = t0 + rr0 + u * kRowStep;
            const int v = FILT ? a.rowidx[min(pos, row1 - 1)] : (int)pos;
            rid[u] = pos < row1 ? v : -1;
            PX_DCHECK(a.dbg, kDbgFlat, pos >= row1 || (v >= 0 && v < a.rows));
        }
        const int64_t pos = t0 + tid;
        const int v = FILT ? a.rowidx[min(pos, row1 - 1)] : (int)pos;
        pid = (tid < kTileRows && pos < row1) ? v : -1;
    };
    float4 pf[kPF];
    float pn = 0.f;
    unsigned pvalid = 0;
    auto fetch = [&](int c) {
        const int f4r = min(kChunk, a.dp - c * kChunk) >> 2;
        pvalid = 0;
#pragma unroll
        for (int u = 0; u < kPF; ++u) {
            pf[u] = *reinterpret_cast<const float4*>(
                a.corpus + (int64_t)max(rid[u], 0) * a.dp + c * kChunk + min(cc, f4r - 1) * 4);
            pvalid |= (rid[u] >= 0 && cc < f4r) ? 1u << u : 0u;
        }
        if (L2) {
            pn = a.norms[max(pid, 0)];
            pvalid |= pid >= 0 ? 1u << kPF : 0u;
        }
    };
    auto commit = [&](int sb, int c, int tp) {
        char* tb = reinterpret_cast<char*>(tile[sb]);
#pragma unroll
        for (int u = 0; u < kPF; ++u)
            *reinterpret_cast<float4*>(tb + (rr0 + u * kRowStep) * (kLdsStride * 4) + cc * 16) =
                zero_unless((pvalid >> u) & 1u, pf[u]);
        if (L2 && c == 0 && tid < kTileRows) tnorm[tp][tid] = (pvalid >> kPF) & 1u ? pn : 0.f;
    };
    auto next_stage = [&](int c, int64_t t, int& cn, int64_t& tn) {
        cn = c + 1 == NCH ? 0 : c + 1;
        tn = cn == 0 ? t + 1 : t;
    };

    if (nstages > 0) {
        tile_ids(0);
        fetch(0);
        commit(0, 0, 0);
        int c1, c2;
        int64_t t1, t2;
        next_stage(0, 0, c1, t1);
        next_stage(c1, t1, c2, t2);
        tile_ids(t1);
        fetch(c1);
        commit(1, c1, (int)(t1 & (kNorms - 1)));
        tile_ids(t2);
    }
    if (tid < 8) committed[tid] = 1;
    __syncthreads();
    const unsigned caddr = (unsigned)(uintptr_t)(committed + (lane & 7));

    // a wave whose 16 queries are all padding only helps stage the rows
    if (qt * (WAVES * QW) + wave * QW >= a.nq) {
        int c = 0;
        int64_t t = 0;
        int rb = 0;
        for (int64_t s = 0; s < nstages; ++s) {
            int c1, c2, c3;
            int64_t t1, t2, t3;
            next_stage(c, t, c1, t1);
            next_stage(c1, t1, c2, t2);
            next_stage(c2, t2, c3, t3);
            fetch(c2);
            tile_ids(t3);
            if (stage_wait(caddr, (int)(s + 1), a.spin_limit) >= a.spin_limit && a.spin_fail &&
                lane == 0)
                atomicOr(a.spin_fail, 1);
            commit(rb == 0 ? 2 : rb - 1, c2, (int)(t2 & (kNorms - 1)));
            stage_publish(committed, wave, lane, (int)(s + 2));
            rb = rb == 2 ? 0 : rb + 1;
            c = c1;
            t = t1;
        }
        return;
    }

    f32x4v acc[4];
    int c = 0;
    int64_t ti = 0;
    int rb = 0;
    for (int64_t s = 0; s < nstages; ++s) {
        int c1, c2, c3;
        int64_t t1, t2, t3;
        next_stage(c, ti, c1, t1);
        next_stage(c1, t1, c2, t2);
        next_stage(c2, t2, c3, t3);
        const int64_t t0 = row0 + ti * kTileRows;
        int gt_raw = kTotalKeyInf;
        if (!COLLECT && c == NCH - 1)
            gt_raw = __hip_atomic_load(gtau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        fetch(c2);
        tile_ids(t3);
        if (c == 0) {
#pragma unroll
            for (int b = 0; b < 4; ++b) acc[b] = (f32x4v){0.f, 0.f, 0.f, 0.f};
        }
        // 16-dim groups holding real dims (the tile is zero past them, and so are the
        // queries' registers)
        const int ng = FULL ? 8 : (min(kChunk, a.dp - c * kChunk) + 15) >> 4;
        const float* tb = tile[rb] + j * kLdsStride + 4 * d;
        auto mfma_chunk = [&](const float4 (&bc)[8]) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (FULL || u < ng) {
                    float4 av[4];
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        av[b] = *reinterpret_cast<const float4*>(tb + 16 * b * kLdsStride + 16 * u);
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[b].x, bc[u].x, acc[b], 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[b].y, bc[u].y, acc[b], 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[b].z, bc[u].z, acc[b], 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[b].w, bc[u].w, acc[b], 0, 0, 0);
                }
            }
        };
        if (c == 0) mfma_chunk(bq[0]);
        else if (NCH == 2 || c == 1) mfma_chunk(bq[1]);
        else mfma_chunk(bq[NCH - 1]);

        // every wave has committed stage s + 1, then this wave's part of stage s + 2
        if (stage_wait(caddr, (int)(s + 1), a.spin_limit) >= a.spin_limit && a.spin_fail &&
            lane == 0)
            atomicOr(a.spin_fail, 1);
        commit(rb == 0 ? 2 : rb - 1, c2, (int)(t2 & (kNorms - 1)));
        stage_publish(committed, wave, lane, (int)(s + 2));
        // the epilogue after the commit: one wave's insertions then hold up no other wave's
        // next stage
        if (c == NCH - 1) {
            // keys of this lane's 16 rows (row 16 b + 4 d + r in key[4 b + r]); L2 drops the
            // per-query ||q||^2 as flat_scan_kernel does
            const float* tn = tnorm[ti & (kNorms - 1)];
            float key[16];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                float4 nv = make_float4(0.f, 0.f, 0.f, 0.f);
                if (L2) nv = *reinterpret_cast<const float4*>(tn + 16 * b + 4 * d);
                const float nn[4] = {nv.x, nv.y, nv.z, nv.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) key[4 * b + r] = L2 ? acc[b][r] + nn[r] : acc[b][r];
            }
            const int rem = (int)min<int64_t>(row1 - t0, (int64_t)kTileRows);
            if constexpr (COLLECT) {
                // every row at or below the threshold (key, then position) is appended
                if (rem < kTileRows) {
#pragma unroll
                    for (int x = 0; x < 16; ++x)
                        key[x] = 16 * (x >> 2) + 4 * d + (x & 3) < rem ? key[x]
                                                                     : __int_as_float(0x7fc00000);
                }
                float kmin = kInf;
#pragma unroll
                for (int x = 0; x < 16; ++x) kmin = fminf(kmin, key[x]);
                if (__ballot(kmin <= cthr)) {
                    const int64_t region =
                        (((int64_t)slot * a.splits + split) * 2 + (d >> 1)) * a.cap;
#pragma unroll
                    for (int x = 0; x < 16; ++x) {
                        const int pos = (int)(t0 + 16 * (x >> 2) + 4 * d + (x & 3));
                        const bool p = key[x] < cthr || (key[x] == cthr && pos <= cpos);
                        const unsigned long long m = __ballot(p);
                        if (m) {
                            const bool pp = (m >> (lane ^ 16)) & 1ull;  // the region's other lane
                            const int at = ccount + ((d & 1) && pp ? 1 : 0);
                            if (p && at < a.cap) {
                                PX_DCHECK(a.dbg, kDbgFlat, qvalid && pos < a.n_eff);
                                a.cand_keys[region + at] = key[x];
                                a.cand_pos[region + at] = pos;
                            }
                            ccount += (p ? 1 : 0) + (pp ? 1 : 0);
                        }
                    }
                }
            } else {
            if (ti == next_refresh) {
                int v[16];
                load_slots16(gbest, a.gbest_ld, h, v);
                gbound = fminf(gbound, from_total_key(kth_smallest32(v, pub_rank)));
                next_refresh = ti + max<int64_t>(1, ti >> 1);
            }
            const float thr = qvalid ? fminf(fminf(tau_k, from_total_key(gt_raw)), gbound) : -kInf;
            if (t0 == row0) {
                // first tile: the query's best kl of its four lanes' 16 rows each, in
                // ascending (key, row) order, one extraction a slot
                constexpr int kNoKey = 0x7fffffff;
                int tk[16];
#pragma unroll
                for (int x = 0; x < 16; ++x)
                    tk[x] = (qvalid && 16 * (x >> 2) + 4 * d + (x & 3) < rem) ? total_key(key[x])
                                                                             : kNoKey;
                int last_t = kNoKey, last_i = kIdNone;
                for (int r = 0; r < a.kl; ++r) {
                    int bt = kNoKey, bx = 0;
#pragma unroll
                    for (int x = 0; x < 16; ++x) {
                        const bool lt = tk[x] < bt;
                        bt = lt ? tk[x] : bt;
                        bx = lt ? x : bx;
                    }
                    const int bi = bt == kNoKey ? kIdNone
                                                : (int)(t0 + 16 * (bx >> 2) + 4 * d + (bx & 3));
                    // the smallest (key, row) over the four lanes of the query
                    int wt = bt, wi = bi;
#pragma unroll
                    for (int m = 16; m <= 32; m <<= 1) {
                        const int ot = __shfl_xor(wt, m), oi = __shfl_xor(wi, m);
                        const bool take = ot < wt || (ot == wt && oi < wi);
                        wt = take ? ot : wt;
                        wi = take ? oi : wi;
                    }
                    if (__ballot(wt != kNoKey) == 0) break;  // fewer than kl rows anywhere
                    const bool mine = bt != kNoKey && bt == wt && bi == wi;
#pragma unroll
                    for (int x = 0; x < 16; ++x) tk[x] = (mine && x == bx) ? kNoKey : tk[x];
                    if (d == 0 && wt != kNoKey) {
                        lkeys[wave][j][r] = from_total_key(wt);
                        lids[wave][j][r] = (unsigned short)(wi - (int)row0);
                    }
                    last_t = wt;
                    last_i = r == a.kl - 1 ? wi : kIdNone;
                }
                const bool full = last_i != kIdNone;
                tau_k = full ? from_total_key(last_t) : kInf;
                tau_i = full ? last_i : kIdNone;
                publish();
            } else {
                const bool eq_ok = thr < tau_k || tau_i >= t0;
                // one compare a row, as in flat_scan_kernel (rows past the split's end NaN)
                const float thr2 = eq_ok ? thr : next_below(thr);
                if (rem < kTileRows) {
#pragma unroll
                    for (int x = 0; x < 16; ++x)
                        key[x] = 16 * (x >> 2) + 4 * d + (x & 3) < rem ? key[x]
                                                                     : __int_as_float(0x7fc00000);
                }
                float kmin = kInf;
#pragma unroll
                for (int x = 0; x < 16; ++x) kmin = fminf(kmin, key[x]);
                if (__ballot(kmin <= thr2)) {
#pragma unroll
                    for (int x = 0; x < 16; ++x) {
                        unsigned long long m = __ballot(key[x] <= thr2);
                        while (m) {
                            const int src = __builtin_ctzll(m);
                            m &= m - 1;
                            const float ck = readlane_f(key[x], src);
                            const int cid =
                                (int)(t0 + 16 * (x >> 2) + 4 * ((src >> 4) & 3) + (x & 3));
                            const float tk = readlane_f(tau_k, src);
                            const int tid_ = readlane_i(tau_i, src);
                            if (!cand_less(ck, cid, tk, tid_)) continue;
                            const int ql = src & 15;
                            float nk;
                            int ni;
                            list_insert<KP>(&lkeys[wave][ql][0], &lids[wave][ql][0], (int)row0,
                                            a.kl, ck, cid, nk, ni);
                            if (j == ql) {
                                tau_k = nk;
                                tau_i = ni;
                            }
                        }
                    }
                    publish();
                }
            }
            }  // !COLLECT
        }

        rb = rb == 2 ? 0 : rb + 1;
        c = c1;
        ti = t1;
    }

    if constexpr (COLLECT) {
        // the region's count (past cap when it overflowed: the select sees it), from its even lane
        if (qvalid && (d & 1) == 0)
            a.cand_count[((int64_t)slot * a.splits + split) * 2 + (d >> 1)] = ccount;
        return;
    }
    // this split's lists: part[q][split][0..kl)
    const int qbase = qt * (WAVES * QW) + wave * QW;
    for (int ql = 0; ql < QW; ++ql) {
        const int qq = qbase + ql;
        if (qq >= a.nq) break;
        float* pk = a.part_keys + ((int64_t)qq * a.splits + split) * a.kl;
        int* pi = a.part_ids + ((int64_t)qq * a.splits + split) * a.kl;
        for (int s = lane; s < a.kl; s += 64) {
            pk[s] = lkeys[wave][ql][s];
            pi[s] = id_load(lids[wave][ql][s], (int)row0);
            PX_DCHECK(a.dbg, kDbgFlat, pi[s] == kIdNone || (pi[s] >= row0 && pi[s] < row1));
        }
    }
}

bool list_resident_queries(int kp, int64_t dp) { return kp == 32 && dp > kChunk && dp <= 3 * kChunk; }
int flat_list_queries_per_block(int kp, int64_t dp) {
    return list_resident_queries(kp, dp) ? 128 : flat_queries_per_block(kp);
}

template <int NCH, bool FULL, bool COLLECT>
static void launch_list16q_n(const FlatScanArgs& a, hipStream_t s) {
    const int64_t qtiles = (a.nq + 127) / 128;
    const dim3 grid((unsigned)(a.xcd_major ? (qtiles * a.splits + 7) / 8 * 8 : qtiles * a.splits));
    if (a.metric == 0) {
        if (a.rowidx) hipLaunchKernelGGL((flat_list16q_kernel<true, true, NCH, FULL, COLLECT>), grid, dim3(512), 0, s, a);
        else hipLaunchKernelGGL((flat_list16q_kernel<true, false, NCH, FULL, COLLECT>), grid, dim3(512), 0, s, a);
    } else {
        if (a.rowidx) hipLaunchKernelGGL((flat_list16q_kernel<false, true, NCH, FULL, COLLECT>), grid, dim3(512), 0, s, a);
        else hipLaunchKernelGGL((flat_list16q_kernel<false, false, NCH, FULL, COLLECT>), grid, dim3(512), 0, s, a);
    }
}
template <bool COLLECT>
static void launch_list16q(const FlatScanArgs& a, hipStream_t s) {
    if (a.dp == 3 * kChunk) launch_list16q_n<3, true, COLLECT>(a, s);
    else if (a.dp > 2 * kChunk) launch_list16q_n<3, false, COLLECT>(a, s);
    else if (a.dp == 2 * kChunk) launch_list16q_n<2, true, COLLECT>(a, s);
    else launch_list16q_n<2, false, COLLECT>(a, s);
}
bool collect_resident_queries(int64_t dp) { return dp > kChunk && dp <= 3 * kChunk; }
hipError_t launch_flat_collect16q(const FlatScanArgs& a0, hipStream_t s) {
    const FlatScanArgs a = with_spin_limit(a0);
    if (a.dense || a.corpus_h || !collect_resident_queries(a.dp) || a.gbest)
        return hipErrorInvalidValue;
    launch_list16q<true>(a, s);
    return hipGetLastError();
}

hipError_t launch_flat_scan(const FlatScanArgs& a0, hipStream_t s) {
    const FlatScanArgs a = with_spin_limit(a0);
    if (list_resident_queries(flat_list_capacity(a.kl), a.dp) && !a.corpus_h) {
        launch_list16q<false>(a, s);
        return hipGetLastError();
    }
    switch (flat_list_capacity(a.kl)) {
        case 32: return launch_scan_t<32, flat_waves(32)>(a, s);
        case 56: return launch_scan_t<56, flat_waves(56)>(a, s);
        case 120: return launch_scan_t<120, flat_waves(120)>(a, s);
        default: return launch_scan_t<128, flat_waves(128)>(a, s);
    }
}

// Sum over the 8 lanes of each aligned group of 8 (every lane of the group gets it):
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], then row_half_mirror pairs the two quads.
__device__ __forceinline__ float sum8_lanes(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));
    return v;
}

// Collect scan for at most NQ query slots on the vector ALUs. Workgroup = one split of
// rows_per_split positions, 8 waves. Eight lanes share a row: lane c8 = lane % 8 reads the
// row's 16-byte columns c8, c8 + 8, ... (each load instruction of a wave reads 8 rows x
// 128 contiguous bytes), and the 8 partial dot products are summed across the lanes. Each
// wave takes 8 R rows a step (R per lane group, for more loads in flight); the queries
// sit in LDS and every lane of a row group reads the same address (a broadcast). A row at
// or below a slot's threshold (key, then position) is appended to the slot's region of
// this split through an LDS counter; with dense set, every key goes to cand_keys
// [slot][n_eff] instead (the threshold sample of a few-query batch). H16: the rows are read
// from their fp16 copy (FlatScanArgs::corpus_h, 128-dim rows whose every value is exact in
// fp16), half the bytes, and widened to fp32 in registers: the same values in the same
// arithmetic, so the keys are bit-identical to the fp32 rows'.
template <int NQ, bool L2, bool FILT, bool H16>
__global__ __launch_bounds__(512) void flat_vcollect_kernel(FlatScanArgs a) {
    extern __shared__ __attribute__((aligned(16))) float sq[];  // [NQ][dp]
    __shared__ float s_thr[NQ];
    __shared__ int s_tpos[NQ], s_cnt[NQ];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = lane & 7, rsub = lane >> 3;
    const int split = blockIdx.x;
    const int64_t row0 = (int64_t)split * a.rows_per_split;
    const int64_t row1 = min(a.n_eff, row0 + a.rows_per_split);
    const int dp = a.dp;
    for (int x = tid; x < NQ * dp; x += blockDim.x) {
        const int sl = x / dp;
        float v = 0.f;
        if (sl < a.nq) {
            const int q = a.qlist ? a.qlist[sl] : sl;
            v = a.queries[(int64_t)q * dp + (x - sl * dp)];
        }
        sq[x] = v;
    }
    if (tid < NQ) {
        float thr = -__int_as_float(0x7f800000);  // padding slots: nothing passes
        int tpos = -1;
        if (tid < a.nq && !a.dense) {  // dense mode has no thresholds
            const int q = a.qlist ? a.qlist[tid] : tid;
            thr = from_total_key(a.thr_key[q]);
            tpos = a.thr_pos[q];
        }
        s_thr[tid] = thr;
        s_tpos[tid] = tpos;
        s_cnt[tid] = 0;
    }
    __syncthreads();

    // R rows per lane group a step: four with one or two slots, fewer with more (registers)
    constexpr int R = NQ <= 2 ? 4 : (NQ <= 8 ? 2 : 1);
    for (int64_t r = row0 + wave * (8 * R); r < row1; r += 8 * R * 8) {
        int64_t pr[R];
        bool vr[R];
        int ir[R];
        const float* xr[R];
        const unsigned short* xh[R];
        float d[R][NQ];
#pragma unroll
        for (int u = 0; u < R; ++u) {
            pr[u] = r + 8 * u + rsub;
            vr[u] = pr[u] < row1;
            const int64_t pp = vr[u] ? pr[u] : row0;
            ir[u] = FILT ? a.rowidx[pp] : (int)pp;
            xr[u] = a.corpus + (int64_t)ir[u] * dp;
            xh[u] = H16 ? a.corpus_h + (int64_t)ir[u] * kChunk : nullptr;
#pragma unroll
            for (int qq = 0; qq < NQ; ++qq) d[u][qq] = 0.f;
        }
#pragma unroll 4
        for (int c = c8 * 4; c < dp; c += 32) {
            // the corpus is read once: nontemporal loads keep it from evicting the rest
            f32x4v v[R];
#pragma unroll
            for (int u = 0; u < R; ++u) {
                if constexpr (H16) {
                    const f16x4v w =
                        __builtin_nontemporal_load(reinterpret_cast<const f16x4v*>(xh[u] + c));
                    v[u] = f32x4v{(float)w[0], (float)w[1], (float)w[2], (float)w[3]};
                } else {
                    v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(xr[u] + c));
                }
            }
#pragma unroll
            for (int qq = 0; qq < NQ; ++qq) {
                const float4 qv = *reinterpret_cast<const float4*>(sq + qq * dp + c);
#pragma unroll
                for (int u = 0; u < R; ++u) {
                    d[u][qq] = __builtin_fmaf(v[u].x, qv.x, d[u][qq]);
                    d[u][qq] = __builtin_fmaf(v[u].y, qv.y, d[u][qq]);
                    d[u][qq] = __builtin_fmaf(v[u].z, qv.z, d[u][qq]);
                    d[u][qq] = __builtin_fmaf(v[u].w, qv.w, d[u][qq]);
                }
            }
        }
        float nr[R];
#pragma unroll
        for (int u = 0; u < R; ++u) nr[u] = L2 ? a.norms[ir[u]] : 0.f;
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq) {
            if (qq >= a.nq) break;
            // lane c8 == u of each row group tests row u (every lane holds the sums)
            float kmine = 0.f;
            int64_t pmine = 0;
            bool vmine = false;
#pragma unroll
            for (int u = 0; u < R; ++u) {
                const float su = sum8_lanes(d[u][qq]);
                // L2 drops ||q||^2, as the MFMA scan does: key = ||x||^2 - 2 q.x; IP: -q.x
                const float ku = L2 ? __builtin_fmaf(-2.0f, su, nr[u]) : -su;
                if (c8 == u) {
                    kmine = ku;
                    pmine = pr[u];
                    vmine = vr[u];
                }
            }
            if (a.dense) {
                // every key, row-major [slot][n_eff]
                if (c8 < R && vmine) a.cand_keys[(int64_t)qq * a.n_eff + pmine] = kmine;
                continue;
            }
            const float thr = s_thr[qq];
            const int tpos = s_tpos[qq];
            if (c8 < R && vmine && (kmine < thr || (kmine == thr && pmine <= tpos))) {
                const int at = atomicAdd(&s_cnt[qq], 1);
                if (at < a.cap) {
                    const int64_t o = ((int64_t)qq * a.splits + split) * a.cap + at;
                    a.cand_keys[o] = kmine;
                    a.cand_pos[o] = (int)pmine;
                }
            }
        }
    }
    __syncthreads();
    if (!a.dense && tid < a.nq) a.cand_count[(int64_t)tid * a.splits + split] = s_cnt[tid];
}

template <int NQ, bool H16>
static void launch_vcollect_h(const FlatScanArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)a.splits), block(512);
    const size_t lds = sizeof(float) * NQ * a.dp;  // at most 64 KB (checked by the caller)
    if (a.metric == 0) {
        if (a.rowidx) hipLaunchKernelGGL((flat_vcollect_kernel<NQ, true, true, H16>), grid, block, lds, s, a);
        else hipLaunchKernelGGL((flat_vcollect_kernel<NQ, true, false, H16>), grid, block, lds, s, a);
    } else {
        if (a.rowidx) hipLaunchKernelGGL((flat_vcollect_kernel<NQ, false, true, H16>), grid, block, lds, s, a);
        else hipLaunchKernelGGL((flat_vcollect_kernel<NQ, false, false, H16>), grid, block, lds, s, a);
    }
}

template <int NQ>
static void launch_vcollect_n(const FlatScanArgs& a, hipStream_t s) {
    if (a.corpus_h) launch_vcollect_h<NQ, true>(a, s);
    else launch_vcollect_h<NQ, false>(a, s);
}

hipError_t launch_flat_vcollect(const FlatScanArgs& a, hipStream_t s) {
    // the slot count rounds up to a power of two: that many query rows of LDS
    int np = 1;
    while (np < a.nq) np <<= 1;
    if (a.nq < 1 || a.nq > kVecQueries || a.dp > kVecMaxDp ||
        (int64_t)np * a.dp > kVecMaxQueryFloats || (a.corpus_h && a.dp != kChunk))
        return hipErrorInvalidValue;
    if (a.nq == 1) launch_vcollect_n<1>(a, s);
    else if (a.nq == 2) launch_vcollect_n<2>(a, s);
    else if (a.nq <= 4) launch_vcollect_n<4>(a, s);
    else if (a.nq <= 8) launch_vcollect_n<8>(a, s);
    else launch_vcollect_n<16>(a, s);
    return hipGetLastError();
}

hipError_t launch_flat_collect_v1(const FlatScanArgs& a0, hipStream_t s) {
    const FlatScanArgs a = with_spin_limit(a0);
    constexpr int kWaves = 8;
    const int64_t qtiles = (a.nq + 32 * kWaves - 1) / (32 * kWaves);
    const bool multi = a.dp > kChunk;
    // several chunks: the grid is padded to a multiple of the 8 XCDs (see flat_scan_kernel)
    const bool xm = multi && a.xcd_major;
    const dim3 grid((unsigned)(xm ? (qtiles * a.splits + 7) / 8 * 8 : qtiles * a.splits)),
        block(kWaves * 64);
    if (a.metric == 0) {
        if (multi) {
            if (a.rowidx) hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, true, true, true, true>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, true, true, false, true>), grid, block, 0, s, a);
        } else {
            if (a.rowidx) hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, true, false, true, true>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, true, false, false, true>), grid, block, 0, s, a);
        }
    } else {
        if (multi) {
            if (a.rowidx) hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, false, true, true, true>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, false, true, false, true>), grid, block, 0, s, a);
        } else {
            if (a.rowidx) hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, false, false, true, true>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((flat_scan_kernel<1, kWaves, false, false, false, true>), grid, block, 0, s, a);
        }
    }
    return hipGetLastError();
}

__global__ void sample_rows_kernel(const int* rowidx, int64_t count, int64_t n_eff, int* row) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const int64_t p = i * n_eff / count;  // < n_eff; i * n_eff < 2^14 * 2^31
    row[i] = rowidx ? rowidx[p] : (int)p;
}

hipError_t launch_sample_rows(const int* rowidx, int64_t count, int64_t n_eff, int* row,
                              hipStream_t s) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(sample_rows_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s,
                       rowidx, count, n_eff, row);
    return hipGetLastError();
}

__global__ void fill_int_kernel(int* p, int64_t n, int v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

hipError_t launch_fill_int(int* p, int64_t n, int v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_int_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

// Device ints to mapped pinned host memory by plain stores (a stream-ordered read-back that
// takes no copy engine).
__global__ void copy_to_host_kernel(const int* src, int* dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

hipError_t launch_copy_to_host(const int* src, int* host_dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(copy_to_host_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       src, host_dst, n);
    return hipGetLastError();
}

// In-LDS bitonic sort (ascending by (key total-order, id)) of p = 2^x entries. A stage of
// stride 64 or more exchanges through LDS between barriers; the stages of stride below 64
// pair entries whose indices differ only in their low six bits, and entry x is handled by
// thread x % blockDim (a multiple of 64), so they pair lanes of one wave: each run of them
// is one pass in registers with cross-lane shuffles. 1,024 entries: 16 barriers, not 56.
__device__ void bitonic_sort(float* sk, int* si, int p) {
    const int nt = blockDim.x, t = threadIdx.x;
    const float kInf = __int_as_float(0x7f800000);
    // merge sizes size_from .. size_to, each with its strides below 64 (entries past p are
    // padding that no entry below p pairs with)
    auto reg_pass = [&](int size_from, int size_to) {
        for (int base = 0; base < p; base += nt) {
            const int x = base + t;
            const bool live = x < p;
            float k = live ? sk[x] : kInf;
            int id = live ? si[x] : kIdNone;
            for (int size = size_from; size <= size_to; size <<= 1) {
                const bool asc = (x & size) == 0;
                for (int st = min(size >> 1, 32); st > 0; st >>= 1) {
                    const float ko = __shfl_xor(k, st);
                    const int io = __shfl_xor(id, st);
                    // the lower entry of an ascending pair keeps the smaller (and so on)
                    const bool other_less = cand_less(ko, io, k, id);
                    if (((x & st) == 0) == asc ? other_less : !other_less) {
                        k = ko;
                        id = io;
                    }
                }
            }
            if (live) {
                sk[x] = k;
                si[x] = id;
            }
        }
    };
    __syncthreads();
    reg_pass(2, min(p, 64));
    for (int size = 128; size <= p; size <<= 1) {
        for (int stride = size >> 1; stride >= 64; stride >>= 1) {
            __syncthreads();
            for (int x = t; x < (p >> 1); x += nt) {
                const int lo = 2 * x - (x & (stride - 1));
                const int hi = lo + stride;
                const bool asc = (lo & size) == 0;
                const float kl = sk[lo], kh = sk[hi];
                const int il = si[lo], ih = si[hi];
                if (cand_less(kh, ih, kl, il) == asc) {
                    sk[lo] = kh; si[lo] = ih;
                    sk[hi] = kl; si[hi] = il;
                }
            }
        }
        __syncthreads();
        reg_pass(size, size);
    }
    __syncthreads();
}

// Candidates a bounded merge sorts at most; more at or below the bound (ties at the bound)
// and the merge sorts all of them.
constexpr int kMergeFiltered = 256;

// One workgroup per query: sort the split candidates, keep the best kl, re-rank them
// exactly (flat), sort again and emit the best k with the reference's finishing and
// padding (flat.rs:229-237; gpu.rs:80-93 for raw keys). With a bound, only candidates at or
// below it are sorted (usually about kl of them): no candidate above a full split list's
// tail can be among the best kl. PQ lists publish no bounds; their kl-th smallest list
// head serves instead.
__global__ __launch_bounds__(1024) void flat_merge_kernel(MergeArgs a) {
    if (a.abort || a.spin_fail) {
        const int v = a.abort ? *a.abort : 0;
        const int sf = a.spin_fail ? *a.spin_fail : 0;
        if (a.verdict && blockIdx.x == 0 && threadIdx.x == 0) {
            a.verdict[0] = v;
            a.verdict[1] = sf;
        }
        if ((a.abort && v == a.abort_seq) || sf) return;
    }
    extern __shared__ __attribute__((aligned(16))) char msmem[];
    __shared__ int s_n;
    int p = 1;
    while (p < a.width) p <<= 1;
    float* sk = reinterpret_cast<float*>(msmem);
    int* si = reinterpret_cast<int*>(sk + p);
    float* rk = reinterpret_cast<float*>(si + p);
    int* ri = reinterpret_cast<int*>(rk + kMaxList);

    const int q = blockIdx.x;
    const float kInf = __int_as_float(0x7f800000);
    const float* pk = a.part_keys + (int64_t)q * a.width;
    const int* pi = a.part_ids + (int64_t)q * a.width;
    // this thread's first kPre candidates, loaded while the bounds load (the filter below
    // takes them from registers)
    constexpr int kPre = 8;
    float pkv[kPre];
    int piv[kPre];
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
        const int x = threadIdx.x + u * blockDim.x;
        pkv[u] = x < a.width ? pk[x] : kInf;
        piv[u] = x < a.width ? pi[x] : kIdNone;
    }
    int bound = a.bound ? a.bound[q] : kTotalKeyInf;
    if (a.gbest) {
        __shared__ int s_gb[32], s_kth;
        const int t = threadIdx.x;
        if (t < 32) s_gb[t] = a.gbest[(int64_t)t * a.gbest_ld + q];
        __syncthreads();
        const int pm = (a.kl + min(a.splits, 32) - 1) / min(a.splits, 32);
        const int rank = (a.kl + pm - 1) / pm;  // <= min(splits, 32)
        if (t < 32) {
            // position of slot t in (key, slot) order; exactly one slot has rank - 1
            const int v = s_gb[t];
            int below = 0;
            for (int u = 0; u < 32; ++u) below += s_gb[u] < v || (s_gb[u] == v && u < t);
            if (below == rank - 1) s_kth = v;
        }
        __syncthreads();
        bound = min(bound, s_kth);
    }
    if (a.sorted_lists && !a.bound && !a.gbest && a.width / a.kl >= a.kl) {
        // kl distinct lists each hold a candidate at or below the kl-th smallest head
        const int nl = a.width / a.kl;
        int ph = 1;
        while (ph < nl) ph <<= 1;
        for (int x = threadIdx.x; x < ph; x += blockDim.x) {
            sk[x] = x < nl ? pk[(int64_t)x * a.kl] : kInf;
            si[x] = x;
        }
        bitonic_sort(sk, si, ph);
        bound = total_key(sk[a.kl - 1]);
        __syncthreads();  // every thread has read it before sk is reused
    }
    int n = -1;  // candidates compacted below the bound; -1: sort them all
    if (bound != kTotalKeyInf) {
        if (threadIdx.x == 0) s_n = 0;
        __syncthreads();
        auto keep = [&](float kv, int id) __attribute__((always_inline)) {
            if (id != kIdNone && total_key(kv) <= bound) {
                const int at = atomicAdd(&s_n, 1);
                if (a.rowidx) id = a.rowidx[id];
                PX_DCHECK(a.dbg, kDbgFlat, at < p && id >= 0);
                sk[at] = kv;  // at < width <= p
                si[at] = id;
            }
        };
#pragma unroll
        for (int u = 0; u < kPre; ++u) keep(pkv[u], piv[u]);
        for (int x = threadIdx.x + kPre * blockDim.x; x < a.width; x += blockDim.x)
            keep(pk[x], pi[x]);
        __syncthreads();
        n = s_n;
        if (n > kMergeFiltered) n = -1;
    }
    int ps = p;  // entries sorted
    if (n >= 0) {
        ps = 1;
        while (ps < n || ps < a.kl) ps <<= 1;
        ps = min(ps, p);
        for (int x = n + threadIdx.x; x < ps; x += blockDim.x) {
            sk[x] = kInf;
            si[x] = kIdNone;
        }
    } else {
        for (int x = threadIdx.x; x < p; x += blockDim.x) {
            float kv = kInf;
            int id = kIdNone;
            if (x < a.width) {
                kv = pk[x];
                id = pi[x];
                if (id != kIdNone && a.rowidx) id = a.rowidx[id];
            }
            sk[x] = kv;
            si[x] = id;
        }
    }
    bitonic_sort(sk, si, ps);

    int p2 = 1;
    while (p2 < a.kl) p2 <<= 1;
    // exact keys: eight lanes per candidate (ref_key_g8)
    for (int x = threadIdx.x >> 3; x < p2; x += blockDim.x >> 3) {
        float kv = kInf;
        int id = kIdNone;
        if (x < a.kl && x < ps) {
            id = si[x];
            kv = sk[x];
            if (id != kIdNone && a.corpus) {
                const float* qv = a.queries + (int64_t)q * a.dp;
                const float* xv = a.corpus + (int64_t)id * a.dp;
                const int gl = threadIdx.x & 7;
                kv = a.metric == 0 ? ref_key_g8(qv, xv, a.dim, true, gl)
                                   : -ref_key_g8(qv, xv, a.dim, false, gl);
            }
            if (id == kIdNone) kv = kInf;
        }
        if ((threadIdx.x & 7) == 0) {
            rk[x] = kv;
            ri[x] = id;
        }
    }
    bitonic_sort(rk, ri, p2);

    for (int x = threadIdx.x; x < a.k; x += blockDim.x) {
        int64_t id = -1;
        float d;
        if (x < p2 && ri[x] != kIdNone) {
            id = ri[x];
            const float kv = rk[x];
            d = a.raw_keys ? kv : (a.metric == 0 ? sqrtf(kv) : -kv);
        } else {
            d = a.raw_keys ? FLT_MAX : (a.metric == 0 ? FLT_MAX : -FLT_MAX);
        }
        a.out_ids[(int64_t)q * a.k + x] = id;
        a.out_dists[(int64_t)q * a.k + x] = d;
    }
}

hipError_t launch_merge(const MergeArgs& a, hipStream_t s) {
    int p = 1;
    while (p < a.width) p <<= 1;
    const size_t lds = (size_t)p * 8 + (size_t)kMaxList * 8;
    static bool big_lds = false;  // widths past 8k candidates need more than 64 KB of LDS
    if (lds > 65536 && !big_lds) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(flat_merge_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)((size_t)kMaxMerge * 8 + kMaxList * 8));
        if (e != hipSuccess) return e;
        big_lds = true;
    }
    // long sorts (many splits: small batches spread over the whole GPU) get 1,024 threads
    const int threads = p >= 4096 ? 1024 : 256;
    hipLaunchKernelGGL(flat_merge_kernel, dim3((unsigned)a.nq), dim3(threads), lds, s, a);
    return hipGetLastError();
}

// One workgroup per query slot of a collect scan. With every candidate stored and at least
// kk of them (or every row a candidate), it finishes the query as flat_merge_kernel does:
// sort by (key, position), re-rank the best kk exactly, sort, emit k. Otherwise it sets the
// query's next threshold and status 1:
//   too few (fewer than kk rows at or below the threshold): the next, looser rung;
//   too many (a region or the LDS overflowed): the kk-th smallest of the candidates it
//   holds (at least kk + 1 of them: the threshold drops below at least one candidate, and
//   at least kk rows stay at or below it).
__global__ __launch_bounds__(1024) void flat_collect_select_kernel(CollectSelectArgs a) {
    if (a.spin_fail && *a.spin_fail) return;
    extern __shared__ __attribute__((aligned(16))) char csmem[];
    float* sk = reinterpret_cast<float*>(csmem);
    int* si = reinterpret_cast<int*>(sk + a.lcap);
    __shared__ int s_off[kMaxCollectRegions + 1];
    __shared__ int s_total, s_over, s_dmin;

    const int b = blockIdx.x;
    const int q = a.qlist ? a.qlist[b] : b;
    const int* cnt = a.cand_count + (int64_t)b * a.regions;
    const float* rk = a.cand_keys + (int64_t)b * a.regions * a.cap;
    const int* rp = a.cand_pos + (int64_t)b * a.regions * a.cap;
    const float kInf = __int_as_float(0x7f800000);
    // region offsets in LDS: each thread sums a run of regions, a block scan places them
    __shared__ int s_wsum[16];
    const int nt = blockDim.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
    if (t == 0) {
        s_total = 0;
        s_over = 0;
        s_dmin = kTotalKeyInf;
    }
    const int per = (a.regions + nt - 1) / nt;
    const int rb0 = min(t * per, a.regions), rb1 = min(rb0 + per, a.regions);
    int my_stored = 0, my_total = 0, my_over = 0;
    // smallest dropped key of the overflowing regions (INT_MIN: unknown)
    int my_dmin = kTotalKeyInf;
    for (int r = rb0; r < rb1; ++r) {
        const int c = cnt[r];
        my_total += c;
        my_stored += min(c, a.cap);
        if (c > a.cap) {
            my_over = 1;
            my_dmin = min(my_dmin, a.cand_dmin ? a.cand_dmin[(int64_t)b * a.regions + r]
                                               : INT_MIN);
        }
    }
    int incl = my_stored;
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
    }
    if (lane == 63) s_wsum[wv] = incl;
    __syncthreads();
    int excl = incl - my_stored;
    for (int w = 0; w < wv; ++w) excl += s_wsum[w];
    for (int r = rb0; r < rb1; ++r) {
        s_off[r] = min(excl, a.lcap);
        excl += min(cnt[r], a.cap);
    }
    if (t == nt - 1) s_off[a.regions] = min(excl, a.lcap);
    if (my_total) atomicAdd(&s_total, my_total);
    if (my_over) {
        atomicOr(&s_over, 1);
        atomicMin(&s_dmin, my_dmin);
    }
    __syncthreads();
    // the kept candidates past the LDS (then some are not held)
    const bool lds_over = excl > a.lcap && t == nt - 1;
    if (lds_over) s_over = 2;
    __syncthreads();
    const int total = s_total;
    const int held = s_off[a.regions];  // candidates loaded into LDS (all kept ones unless
                                        // s_over == 2)
    const bool all_rows = a.thr_key[q] == kTotalKeyInf;
    // s_over: 0 none, 1 a region overflowed (every kept candidate held), 2 past the LDS.
    // With 1 the query finishes if its kk-th smallest held key is below every dropped key
    // (s_dmin), decided once they are sorted: no dropped row can be among its best kk.
    const int over = s_over;
    const bool may_finish = over == 0 || (over == 1 && s_dmin != INT_MIN);
    bool finish = over == 0 && (total >= a.kk || all_rows);
    if (over == 0 && !finish) {
        // too few: next rung
        if (threadIdx.x == 0) {
            const int r = a.rung[q] + 1;
            const bool more = r < kRungs;
            a.thr_key[q] = more ? a.ladder_key[(int64_t)q * kRungs + r] : kTotalKeyInf;
            a.thr_pos[q] = more ? a.ladder_pos[(int64_t)q * kRungs + r] : kIdNone;
            a.rung[q] = min(r, kRungs);
            a.status[q] = 1;
        }
        return;
    }
    if (over && held <= a.kk) {
        // too many, but too few held to tighten: the caller collects again with a larger cap
        if (threadIdx.x == 0) a.status[q] = 1;
        return;
    }

    // A finishing query with the scan's shared bound sorts only the candidates at or below
    // it: the kk-th smallest slot (every slot has a collected row of its own at or below it).
    int bound = kTotalKeyInf;
    if (a.gbest && finish) {
        __shared__ int s_gb[32], s_kth;
        if (t < 32) s_gb[t] = a.gbest[(int64_t)t * a.gbest_ld + q];
        if (t == 0) s_kth = kTotalKeyInf;
        __syncthreads();
        if (t < 32) {
            // position of slot t in (key, slot) order; exactly one slot has kk - 1
            const int v = s_gb[t];
            int below = 0;
            for (int u = 0; u < 32; ++u) below += s_gb[u] < v || (s_gb[u] == v && u < t);
            if (below == a.kk - 1) s_kth = v;
        }
        __syncthreads();
        bound = s_kth;
    }
    // Sixteen threads per region read its stored candidates in order (contiguous loads);
    // with a bound, a position is read only for a key at or below it. The regions' LDS
    // ranges (s_off) were clamped to lcap: entries past it are dropped (overflow).
    int avail = held;  // candidates sorted into sk/si
    if (bound != kTotalKeyInf) {
        if (t == 0) s_total = 0;
        __syncthreads();
    }
    for (int r = t >> 4; r < a.regions; r += nt >> 4) {
        const int n_r = s_off[r + 1] - s_off[r];
        PX_DCHECK(a.dbg, kDbgFlat, n_r >= 0 && n_r <= a.cap && s_off[r + 1] <= a.lcap);
        const float* rkr = rk + (int64_t)r * a.cap;
        const int* rpr = rp + (int64_t)r * a.cap;
        for (int c = t & 15; c < n_r; c += 16) {
            const float kv = rkr[c];
            if (bound == kTotalKeyInf) {
                sk[s_off[r] + c] = kv;
                si[s_off[r] + c] = rpr[c];
            } else if (total_key(kv) <= bound) {
                const int i = atomicAdd(&s_total, 1);
                sk[i] = kv;
                si[i] = rpr[c];
            }
        }
    }
    if (bound != kTotalKeyInf) {
        __syncthreads();
        avail = s_total;
    }
    // Many more candidates than the kk it keeps (a threshold round holds two to ten times kk):
    // the kk-th smallest key by a radix select (four 8-bit passes over the order-preserving
    // unsigned form of the total-order key, so the key is exact), then only the candidates
    // at or below it (at least kk, ties included) are compacted and sorted.
    if (avail > 512 && avail > 2 * a.kk) {
        __shared__ unsigned rhist[256];
        __shared__ unsigned s_pre, s_need;
        if (t == 0) {
            s_pre = 0;
            s_need = (unsigned)a.kk;
        }
        for (int pass = 0; pass < 4; ++pass) {
            const int shift = 24 - 8 * pass;  // digit bits [shift, shift + 8)
            for (int x = t; x < 256; x += nt) rhist[x] = 0;
            __syncthreads();
            const unsigned pre = s_pre;
            for (int x = t; x < avail; x += nt) {
                const unsigned u = (unsigned)total_key(sk[x]) ^ 0x80000000u;
                if (pass == 0 || (u >> (shift + 8)) == pre) atomicAdd(&rhist[(u >> shift) & 0xffu], 1u);
            }
            __syncthreads();
            if (t < 64) {
                // lane t holds bins 4t .. 4t + 3; the bin where the count reaches s_need
                unsigned c[4], sum = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    c[e] = rhist[4 * t + e];
                    sum += c[e];
                }
                unsigned incl = sum;
                for (int off = 1; off < 64; off <<= 1) {
                    const unsigned v = __shfl_up(incl, off);
                    if (lane >= off) incl += v;
                }
                const unsigned need = s_need;
                unsigned before = incl - sum;
                int digit = -1;
                unsigned below = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (digit < 0 && before + c[e] >= need) {
                        digit = 4 * t + e;
                        below = before;
                    }
                    before += c[e];
                }
                // some bin reaches it: need <= the keys under the prefix, at least kk at first
                const unsigned long long m = __ballot(digit >= 0);
                const int src = __builtin_ctzll(m);
                const int dsel = __shfl(digit, src);
                const unsigned bsel = __shfl(below, src);
                if (t == 0) {
                    s_pre = (pre << 8) | (unsigned)dsel;
                    s_need = need - bsel;
                }
            }
            __syncthreads();
        }
        const unsigned kth = s_pre;
        // this thread's entries (at most lcap / blockDim = 16), then the survivors to the front
        constexpr int kHeld = kMaxCollect / 1024;
        PX_DCHECK(a.dbg, kDbgFlat, avail <= kHeld * nt);
        float ck[kHeld];
        int ci[kHeld];
#pragma unroll
        for (int u = 0; u < kHeld; ++u) {
            const int x = t + u * nt;
            ck[u] = x < avail ? sk[x] : kInf;
            ci[u] = x < avail ? si[x] : kIdNone;
        }
        if (t == 0) s_total = 0;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kHeld; ++u) {
            const int x = t + u * nt;
            if (x < avail && ((unsigned)total_key(ck[u]) ^ 0x80000000u) <= kth) {
                const int i = atomicAdd(&s_total, 1);
                sk[i] = ck[u];
                si[i] = ci[u];
            }
        }
        __syncthreads();
        avail = s_total;
    }
    int p = 1;
    while (p < avail) p <<= 1;
    for (int x = avail + threadIdx.x; x < p; x += blockDim.x) {
        sk[x] = kInf;
        si[x] = kIdNone;
    }
    bitonic_sort(sk, si, p);
    // a region overflowed: the kk-th smallest held key (held > kk) below every dropped one
    if (over == 1 && may_finish) finish = total_key(sk[a.kk - 1]) < s_dmin;

    if (!finish) {
        // too many: tighten to the kk-th smallest held candidate
        if (threadIdx.x == 0) {
            a.thr_key[q] = total_key(sk[a.kk - 1]);
            a.thr_pos[q] = si[a.kk - 1];
            a.status[q] = 1;
        }
        return;
    }

    const int keep = min(a.kk, avail);
    int p2 = 1;
    while (p2 < keep) p2 <<= 1;
    // exact keys: eight lanes per candidate (ref_key_g8); each candidate's entry is read by
    // its own group only, and written after the group has read it
    for (int x = threadIdx.x >> 3; x < p2; x += blockDim.x >> 3) {
        float kv = kInf;
        int id = kIdNone;
        if (x < keep && si[x] != kIdNone) {
            id = si[x];
            if (a.rowidx) id = a.rowidx[id];
            kv = sk[x];
            if (a.corpus) {
                const float* qv = a.queries + (int64_t)q * a.dp;
                const float* xv = a.corpus + (int64_t)id * a.dp;
                const int gl = threadIdx.x & 7;
                kv = a.metric == 0 ? ref_key_g8(qv, xv, a.dim, true, gl)
                                   : -ref_key_g8(qv, xv, a.dim, false, gl);
            }
        }
        if ((threadIdx.x & 7) == 0) {
            sk[x] = kv;
            si[x] = id;
        }
    }
    bitonic_sort(sk, si, p2);
    for (int x = threadIdx.x; x < a.k; x += blockDim.x) {
        int64_t id = -1;
        float d;
        if (x < keep && si[x] != kIdNone) {
            id = si[x];
            const float kv = sk[x];
            d = a.raw_keys ? kv : (a.metric == 0 ? sqrtf(kv) : -kv);
        } else {
            d = a.raw_keys ? FLT_MAX : (a.metric == 0 ? FLT_MAX : -FLT_MAX);
        }
        a.out_ids[(int64_t)q * a.k + x] = id;
        a.out_dists[(int64_t)q * a.k + x] = d;
    }
    if (threadIdx.x == 0) a.status[q] = 0;
}

// One workgroup of 1024 threads per query: its sampled keys in registers (up to 24 per
// thread, row q of the row-major keys), three 8-bit radix passes over the top 24 bits of
// the order-preserving unsigned form of the total-order key, both ranks at once (LDS
// histograms of 256 bins each); the 8 bits below are taken as ones, so each threshold is
// the top of the bin that holds its rank.
__global__ __launch_bounds__(1024) void flat_ladder_kernel(LadderArgs a) {
    constexpr int kPer = kMaxLadderEntries / 1024;
    constexpr unsigned kNone = 0xffffffffu;
    constexpr int kWaves = 16;
    // the first pass counts every key once for both rungs, into one histogram per wave (16
    // waves contending for 256 bins cost more than the sum over waves afterwards); the later
    // passes count only the keys under a rung's prefix, few, straight into the rung's bins
    __shared__ unsigned whist[kWaves][256];
    __shared__ unsigned hist[kRungs][256];
    __shared__ unsigned s_prefix[kRungs], s_rank[kRungs];
    const int q = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const float* base = a.keys + (int64_t)q * a.ld;
    unsigned u[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = t + i * 1024;
        const float kv = e < a.count ? base[e] : __int_as_float(0x7f800000);
        // +inf (rows past a split's end) is left out
        u[i] = kv < __int_as_float(0x7f800000) ? (unsigned)total_key(kv) ^ 0x80000000u : kNone;
    }
    if (t < kRungs) {
        s_prefix[t] = 0;
        s_rank[t] = (unsigned)a.ranks[t];
    }
    for (int x = t; x < kWaves * 256; x += blockDim.x) (&whist[0][0])[x] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (u[i] != kNone) atomicAdd(&whist[wv][u[i] >> 24], 1u);
    __syncthreads();
    for (int x = t; x < 256; x += blockDim.x) {
        unsigned c = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) c += whist[w][x];
#pragma unroll
        for (int r = 0; r < kRungs; ++r) hist[r][x] = c;
    }
    __syncthreads();
    for (int pass = 0; pass < 3; ++pass) {
        const int shift = 24 - 8 * pass;  // digit bits [shift, shift + 8)
        if (pass > 0) {
            for (int x = t; x < kRungs * 256; x += blockDim.x) (&hist[0][0])[x] = 0;
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                if (u[i] == kNone) continue;
                const unsigned d = (u[i] >> shift) & 0xffu;
#pragma unroll
                for (int r = 0; r < kRungs; ++r) {
                    // keys whose higher digits match the rung's prefix so far
                    if ((u[i] >> (shift + 8)) == s_prefix[r]) atomicAdd(&hist[r][d], 1u);
                }
            }
            __syncthreads();
        }
        if (wv < kRungs) {
            // lane holds bins 4 lane .. 4 lane + 3; inclusive scan across the wave
            unsigned c[4], sum = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                c[e] = hist[wv][4 * lane + e];
                sum += c[e];
            }
            unsigned incl = sum;
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned v = __shfl_up(incl, off);
                if (lane >= off) incl += v;
            }
            const unsigned need = s_rank[wv];
            unsigned before = incl - sum;
            // the lane whose bins cross the rank picks the digit
            int digit = -1;
            unsigned below = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (digit < 0 && before + c[e] >= need) {
                    digit = 4 * lane + e;
                    below = before;
                }
                before += c[e];
            }
            const unsigned long long m = __ballot(digit >= 0);
            const int src = m ? __builtin_ctzll(m) : 63;
            const int dsel = __shfl(digit, src);
            const unsigned bsel = __shfl(below, src);
            if (lane == 0) {
                // fewer keys than the rank (not for ranks <= the sample size): +inf
                s_prefix[wv] = m ? (s_prefix[wv] << 8) | (unsigned)dsel : 0xffffffu;
                s_rank[wv] = m ? need - bsel : 1u;
            }
        }
        __syncthreads();
    }
    if (t < kRungs) {
        const unsigned top = (s_prefix[t] << 8) | 0xffu;
        int tk = (int)(top ^ 0x80000000u);
        if (tk > kTotalKeyInf) tk = kTotalKeyInf;  // a bin reaching past +inf: every row passes
        a.ladder_key[(int64_t)q * kRungs + t] = tk;
        a.ladder_pos[(int64_t)q * kRungs + t] = kIdNone;
        if (t == 0) {
            a.thr_key[q] = tk;
            a.thr_pos[q] = kIdNone;
            a.rung[q] = 0;
        }
    }
}

// The ladder of a small sample (at most kSmallLadder keys a query, the seed of a bounded
// round): one wave a query sorts its keys in registers (bitonic, eight a lane) and takes each
// rung's rank-th smallest key exactly, where flat_ladder_kernel's 1,024 threads a query
// would mostly idle (139 us for 10,000 queries of 512 keys). As there, +inf keys are left
// out, a rung past the keys is +inf, and every position at the rung's key passes.
constexpr int kSmallLadder = 512;
__global__ __launch_bounds__(256) void flat_ladder_small_kernel(LadderArgs a) {
    constexpr unsigned kNone = 0xffffffffu;
    const int lane = threadIdx.x & 63;
    const int q = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (q >= a.nq) return;  // whole waves; no barrier below
    const float* base = a.keys + (int64_t)q * a.ld;
    // element n = 8 lane + i of the sorting network in u[i]
    unsigned u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int e = lane + 64 * i;
        const float kv = e < a.count ? base[e] : __int_as_float(0x7f800000);
        u[i] = kv < __int_as_float(0x7f800000) ? (unsigned)total_key(kv) ^ 0x80000000u : kNone;
    }
#pragma unroll
    for (int k = 2; k <= 512; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j >= 8) {
                // partner n ^ j is lane ^ (j / 8), same register; the lower of the two keeps
                // the smaller key where the run ascends ((n & k) == 0)
                const int pl = j >> 3;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const unsigned o = (unsigned)__shfl_xor((int)u[i], pl);
                    const bool asc = ((8 * lane + i) & k) == 0;
                    const bool keep_min = ((lane & pl) == 0) == asc;
                    u[i] = keep_min ? min(u[i], o) : max(u[i], o);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if ((i & j) == 0) {
                        const bool asc = ((8 * lane + i) & k) == 0;
                        const unsigned lo = min(u[i], u[i | j]), hi = max(u[i], u[i | j]);
                        u[i] = asc ? lo : hi;
                        u[i | j] = asc ? hi : lo;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kRungs; ++r) {
        const int n = a.ranks[r] - 1;  // uniform
        unsigned mine = u[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mine = (n & 7) == i ? u[i] : mine;
        const unsigned v = (n >= 0 && n < 512) ? (unsigned)__shfl((int)mine, n >> 3) : kNone;
        const int tk = v == kNone ? kTotalKeyInf : (int)(v ^ 0x80000000u);
        if (lane == 0) {
            a.ladder_key[(int64_t)q * kRungs + r] = tk;
            a.ladder_pos[(int64_t)q * kRungs + r] = kIdNone;
            if (r == 0) {
                a.thr_key[q] = tk;
                a.thr_pos[q] = kIdNone;
                a.rung[q] = 0;
            }
        }
    }
}

hipError_t launch_ladder(const LadderArgs& a, hipStream_t s) {
    if (a.nq <= 0) return hipSuccess;
    if (a.count > kMaxLadderEntries || a.ld < a.count) return hipErrorInvalidValue;
    if (a.count <= kSmallLadder) {
        hipLaunchKernelGGL(flat_ladder_small_kernel, dim3((unsigned)((a.nq + 3) / 4)), dim3(256),
                           0, s, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(flat_ladder_kernel, dim3((unsigned)a.nq), dim3(1024), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_collect_select(const CollectSelectArgs& a, int slots, hipStream_t s) {
    if (slots <= 0) return hipSuccess;
    const size_t lds = (size_t)a.lcap * 8;
    static bool big_lds = false;
    if (lds > 65536 && !big_lds) {
        const hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(flat_collect_select_kernel),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)((size_t)kMaxCollect * 8));
        if (e != hipSuccess) return e;
        big_lds = true;
    }
    // a quarter of the threads while the sorts are short
    const int threads = a.lcap >= 8192 ? 1024 : 256;
    hipLaunchKernelGGL(flat_collect_select_kernel, dim3((unsigned)slots), dim3(threads), lds, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Support kernels
// ---------------------------------------------------------------------------
__global__ void row_norms_kernel(const float* x, int64_t rows, int dp, float* out) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float4* v = reinterpret_cast<const float4*>(x + r * dp);
    float s = 0.f;
    for (int i = 0; i < (dp >> 2); ++i) {
        const float4 t = v[i];
        s = __builtin_fmaf(t.x, t.x, s);
        s = __builtin_fmaf(t.y, t.y, s);
        s = __builtin_fmaf(t.z, t.z, s);
        s = __builtin_fmaf(t.w, t.w, s);
    }
    out[r] = s;
}

hipError_t launch_row_norms(const float* x, int64_t rows, int dp, float* out, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    const int64_t blocks = (rows + 255) / 256;
    hipLaunchKernelGGL(row_norms_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, rows, dp, out);
    return hipGetLastError();
}

__global__ void pad_rows_kernel(const float* src, int64_t rows, int dim, int dp, float* dst) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= rows * dp) return;
    const int64_t r = e / dp;
    const int d = (int)(e - r * dp);
    dst[e] = d < dim ? src[r * dim + d] : 0.f;
}

hipError_t launch_pad_rows(const float* src, int64_t rows, int dim, int dp, float* dst,
                           hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    const int64_t blocks = (rows * dp + 255) / 256;
    hipLaunchKernelGGL(pad_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, rows, dim,
                       dp, dst);
    return hipGetLastError();
}

// *flag = 1 when any of count floats is NaN or infinite (exponent bits all ones), else 0.
__global__ __launch_bounds__(256) void nonfinite_kernel(const float* x, int64_t count, int* flag) {
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x)
        bad |= (__float_as_uint(x[i]) & 0x7f800000u) == 0x7f800000u;
    if (__ballot(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

hipError_t launch_nonfinite_check(const float* x, int64_t count, int* flag, hipStream_t s) {
    hipError_t e = launch_fill_int(flag, 1, 0, s);
    if (e != hipSuccess || count <= 0) return e;
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 2048);
    hipLaunchKernelGGL(nonfinite_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, count, flag);
    return hipGetLastError();
}

// out[i] = x[i] as fp16 bits; *inexact = 1 when any x[i] is not exactly an fp16 zero or
// normal number (a rounded value, past 65504, or below fp16's smallest normal 2^-14: fp16
// subnormals are excluded so that no MFMA input depends on subnormal handling). count is a
// multiple of 4; x and out are 16- and 8-byte aligned.
__global__ __launch_bounds__(256) void to_f16_kernel(const float4* x, int64_t count4,
                                                     ushort4* out, int* inexact, int bit) {
    bool bad = false;
    auto one = [&](float v) -> unsigned short {
        const _Float16 hv = (_Float16)v;
        bad |= !((float)hv == v && (v == 0.f || fabsf(v) >= 0x1p-14f));
        return __builtin_bit_cast(unsigned short, hv);
    };
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float4 v = x[i];
        out[i] = make_ushort4(one(v.x), one(v.y), one(v.z), one(v.w));
    }
    if (__ballot(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(inexact, bit);
}

hipError_t launch_to_f16(const float* x, int64_t count, unsigned short* out, int* inexact,
                         hipStream_t s, int bit) {
    if (count % 4 != 0 || ((uintptr_t)x & 15) != 0 || ((uintptr_t)out & 7) != 0)
        return hipErrorInvalidValue;
    if (count <= 0) return hipSuccess;
    const int64_t count4 = count / 4;
    const int64_t blocks = std::min<int64_t>((count4 + 255) / 256, 4096);
    hipLaunchKernelGGL(to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(x), count4,
                       reinterpret_cast<ushort4*>(out), inexact, bit);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void list_prologue_kernel(const float* x, int64_t count,
                                                            int* flag, int seq, int* gtau,
                                                            int64_t ngtau, int* gbest,
                                                            int64_t ngbest, int* zero) {
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    if (zero && i0 == 0) *zero = 0;
    bool bad = false;
    for (int64_t i = i0; i < count; i += step)
        bad |= (__float_as_uint(x[i]) & 0x7f800000u) == 0x7f800000u;
    for (int64_t i = i0; i < ngtau; i += step) gtau[i] = kTotalKeyInf;
    for (int64_t i = i0; i < ngbest; i += step) gbest[i] = kTotalKeyInf;
    if (__ballot(bad) != 0 && (threadIdx.x & 63) == 0) atomicMax(flag, seq);
}

hipError_t launch_list_prologue(const float* x, int64_t count, int* flag, int seq, int* gtau,
                                int64_t ngtau, int* gbest, int64_t ngbest, int* zero,
                                hipStream_t s) {
    if (count > 0 && !flag) return hipErrorInvalidValue;
    const int64_t most = std::max<int64_t>({count, ngtau, ngbest, (int64_t)1});
    const int64_t blocks = std::min<int64_t>((most + 255) / 256, 2048);
    hipLaunchKernelGGL(list_prologue_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, count,
                       flag, seq, gtau, ngtau, gbest, ngbest, zero);
    return hipGetLastError();
}

// Ordered mask compaction: 4096 mask bytes per block of 256 threads (16 per thread).
constexpr int kCompactPerBlock = 4096;

int64_t mask_compact_scratch(int64_t n) {
    return (n + kCompactPerBlock - 1) / kCompactPerBlock + 1;
}

__global__ __launch_bounds__(256) void mask_count_kernel(const uint8_t* mask, int64_t n,
                                                         int* counts) {
    __shared__ int wsum[4];
    const int64_t base = (int64_t)blockIdx.x * kCompactPerBlock + threadIdx.x * 16;
    int c = 0;
    for (int i = 0; i < 16; ++i)
        if (base + i < n && mask[base + i]) ++c;
    for (int off = 32; off > 0; off >>= 1) c += __shfl_down(c, off);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) counts[blockIdx.x] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

// Exclusive scan of nb block counts in one workgroup; counts[nb] receives the total.
__global__ __launch_bounds__(1024) void mask_scan_kernel(int* counts, int nb, int* d_count) {
    __shared__ int buf[1024];
    __shared__ int carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    for (int base = 0; base < nb; base += 1024) {
        const int i = base + threadIdx.x;
        const int v = i < nb ? counts[i] : 0;
        buf[threadIdx.x] = v;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int t = threadIdx.x >= off ? buf[threadIdx.x - off] : 0;
            __syncthreads();
            buf[threadIdx.x] += t;
            __syncthreads();
        }
        if (i < nb) counts[i] = carry + buf[threadIdx.x] - v;
        __syncthreads();
        if (threadIdx.x == 1023) carry += buf[1023];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        counts[nb] = carry;
        *d_count = carry;
    }
}

__global__ __launch_bounds__(256) void mask_scatter_kernel(const uint8_t* mask, int64_t n,
                                                           const int* offsets, int* rowidx) {
    __shared__ int wsum[4];
    const int64_t base = (int64_t)blockIdx.x * kCompactPerBlock + threadIdx.x * 16;
    int c = 0;
    for (int i = 0; i < 16; ++i)
        if (base + i < n && mask[base + i]) ++c;
    // inclusive scan of c across the workgroup
    int incl = c;
    const int lane = threadIdx.x & 63;
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off);
        if (lane >= off) incl += t;
    }
    if (lane == 63) wsum[threadIdx.x >> 6] = incl;
    __syncthreads();
    int wave_off = 0;
    for (int w = 0; w < (int)(threadIdx.x >> 6); ++w) wave_off += wsum[w];
    int out = offsets[blockIdx.x] + wave_off + incl - c;
    for (int i = 0; i < 16; ++i)
        if (base + i < n && mask[base + i]) rowidx[out++] = (int)(base + i);
}

hipError_t launch_mask_compact(const uint8_t* mask, int64_t n, int* rowidx, int* scratch,
                               int* d_count, hipStream_t s) {
    const int nb = (int)((n + kCompactPerBlock - 1) / kCompactPerBlock);
    if (nb == 0) {
        return hipMemsetAsync(d_count, 0, sizeof(int), s);
    }
    hipLaunchKernelGGL(mask_count_kernel, dim3(nb), dim3(256), 0, s, mask, n, scratch);
    hipLaunchKernelGGL(mask_scan_kernel, dim3(1), dim3(1024), 0, s, scratch, nb, d_count);
    hipLaunchKernelGGL(mask_scatter_kernel, dim3(nb), dim3(256), 0, s, mask, n, scratch, rowidx);
    return hipGetLastError();
}

__global__ void copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

hipError_t launch_copy(const float4* src, float4* dst, int64_t n4, hipStream_t s) {
    hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, s, src, dst, n4);
    return hipGetLastError();
}

}  // namespace px
