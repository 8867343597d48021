// px_pq.hip -- PqIndex ADC scan for gfx950.
//
// Replaces crates/core/src/pq.rs:299-347 (per query: build the m x 2^nbits LUT, sum m
// LUT entries per code row, heap top-k). A workgroup holds the LUTs of QPB queries in
// LDS (built in the reference's exact arithmetic, pq.rs:123-136), interleaved by query
// (lut[sub][code][query]) so that one LDS read gathers the entry of every query for a
// (row, subspace): a 16-byte read for four queries instead of four random 4-byte reads.
// Code rows stream with one coalesced 16-byte load per row (m = 16), and each row's m
// lookups are summed in subspace order starting from +0.0 -- the reference's order
// (pq.rs:320-323), so the keys are bit-identical to the CPU's. Each wave keeps per-query
// sorted lists in LDS; the per-wave lists are merged and finished by flat_merge_kernel
// (no re-rank: exact keys). Work is bounded by code bytes and LUT gathers, not flops: no
// MFMA here.
#include "px_device.h"
#include "px_kernels.h"

namespace px {

constexpr int kPqWaves = 8;
constexpr int kPqThreads = kPqWaves * 64;

int pq_list_capacity(int kl) {
    if (kl <= 16) return 16;
    if (kl <= 32) return 32;
    if (kl <= 64) return 64;
    return 128;
}
int pq_lists_per_split() { return kPqWaves; }
int pq_rows_per_block_step() { return kPqThreads; }

// Queries per workgroup: as many LUTs as fit in 64 KB of LDS, at most 4.
int pq_queries_per_block(int m, int ks) {
    const int lut_bytes = m * ks * 4;
    int qpb = 65536 / (lut_bytes > 0 ? lut_bytes : 1);
    if (qpb >= 4) return 4;
    if (qpb >= 2) return 2;
    return 1;
}

// One code row; aligned so that m = 16 loads as a single dwordx4 and m = 8 as a dwordx2.
template <int M>
struct alignas(M % 16 == 0 ? 16 : (M % 8 == 0 ? 8 : 1)) CodeRow {
    uint8_t c[M];
};

// The entries of QPB queries for one (row, subspace), as one LDS read.
template <int QPB>
struct Entry;
template <>
struct Entry<4> { using type = float4; };
template <>
struct Entry<2> { using type = float2; };
template <>
struct Entry<1> { using type = float; };
template <int QPB>
__device__ __forceinline__ void add_entry(float (&key)[QPB], const typename Entry<QPB>::type& v) {
    if constexpr (QPB == 4) {
        key[0] = key[0] + v.x;
        key[1] = key[1] + v.y;
        key[2] = key[2] + v.z;
        key[3] = key[3] + v.w;
    } else if constexpr (QPB == 2) {
        key[0] = key[0] + v.x;
        key[1] = key[1] + v.y;
    } else {
        key[0] = key[0] + v;
    }
}

// LDS bytes of a launch: the LUTs of QPB queries, then each wave's lists of KP.
static size_t pq_lds_bytes(int qpb, int m, int ks, int kp) {
    return (size_t)qpb * m * ks * sizeof(float) + (size_t)kPqWaves * qpb * kp * 8;
}

// M > 0: compile-time subspace count with a vector code load; M == 0: runtime m. KS > 0:
// compile-time centroid count (the LUT's subspace stride a constant, so each gather's
// subspace offset is the LDS instruction's immediate).
// COLLECT (k past the lists): no lists; each wave appends every row at or below its
// query's threshold (key, position) to its region of (query slot, split, wave), or, with
// a.dense, writes every key to cand_keys[q][n_eff].
//
// The row loop is software-pipelined: a lane's code row for the next iteration (and, with
// a filter, the row id of the one after) is loaded during this one, and a row's M gathers
// are issued together before its M in-order sums, so that a wave keeps M LDS reads and its
// next global load in flight (the gathers' bank conflicts make each cost about twice a
// conflict-free read; latency, not the LDS unit, bounded the loop that waited for each).
template <int QPB, int KP, int M, bool COLLECT = false, int KS = 0>
__global__ __launch_bounds__(kPqThreads) void pq_scan_kernel(PqScanArgs a) {
    // LDS (all of it dynamic, pq_lds_bytes): the LUTs at offset 0, so that a gather's
    // subspace offset (sub * ks * QPB * 4 bytes, at most 61,440) is the LDS instruction's
    // immediate, then the per-wave lists [kPqWaves][QPB][KP] of keys and of ids
    extern __shared__ __attribute__((aligned(16))) float lut[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m = M > 0 ? M : a.m;
    const int ks = KS > 0 ? KS : a.ks;
    const int lut_len = m * ks;
    float* const lkeys = lut + QPB * lut_len;
    int* const lids = reinterpret_cast<int*>(lkeys + kPqWaves * QPB * KP);
    auto list_k = [&](int qq) { return lkeys + (wave * QPB + qq) * KP; };
    auto list_i = [&](int qq) { return lids + (wave * QPB + qq) * KP; };
    const int qg = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
    const int q0 = qg * QPB;
    const float kInf = __int_as_float(0x7f800000);
    // query index of slot q0 + qq (a retry round lists the queries it serves)
    auto qidx = [&](int qq) { return (COLLECT && a.qlist) ? a.qlist[q0 + qq] : q0 + qq; };

    // lut[(sub * ks + c) * QPB + qq] = l2_sqr(q_sub, centroid) | -inner_product(q_sub, centroid)
    for (int x = tid; x < QPB * lut_len; x += kPqThreads) {
        const int qq = x % QPB;
        const int rest = x / QPB;
        const int sub = rest / ks;
        const int c = rest - sub * ks;
        float v = 0.f;
        if (q0 + qq < a.nq) {
            const float* qs = a.queries + (int64_t)qidx(qq) * a.dim + sub * a.dsub;
            const float* cen = a.codebooks + ((int64_t)sub * ks + c) * a.dsub;
            v = a.metric == 0 ? ref_l2_sqr(qs, cen, a.dsub) : -ref_inner_product(qs, cen, a.dsub);
        }
        lut[x] = v;
    }
    if constexpr (!COLLECT) {
        for (int x = lane; x < QPB * KP; x += 64) {
            list_k(x / KP)[x % KP] = kInf;
            list_i(x / KP)[x % KP] = kIdNone;
        }
    }
    __syncthreads();

    float tau_k[QPB];
    int tau_i[QPB];
#pragma unroll
    for (int qq = 0; qq < QPB; ++qq) {
        tau_k[qq] = kInf;
        tau_i[qq] = kIdNone;
    }
    bool qok[QPB];
#pragma unroll
    for (int qq = 0; qq < QPB; ++qq) qok[qq] = q0 + qq < a.nq;
    // collect mode: thresholds (nothing passes -inf) and append counters
    float cthr[QPB];
    int cpos[QPB], ccount[QPB];
#pragma unroll
    for (int qq = 0; qq < QPB; ++qq) {
        cthr[qq] = -kInf;
        cpos[qq] = -1;
        ccount[qq] = 0;
        if (COLLECT && !a.dense && qok[qq]) {
            cthr[qq] = __int_as_float(a.thr_key[qidx(qq)] ^
                                      (int)(((unsigned)(a.thr_key[qidx(qq)] >> 31)) >> 1));
            cpos[qq] = a.thr_pos[qidx(qq)];
        }
    }

    // one row's keys of all QPB queries are ready: select (lists) or collect
    auto consume = [&](int base, int pos, bool valid, float (&key)[QPB])
        __attribute__((always_inline)) {
        if constexpr (COLLECT) {
#pragma unroll
            for (int qq = 0; qq < QPB; ++qq) {
                if (a.dense) {
                    if (valid && qok[qq]) a.cand_keys[(int64_t)(q0 + qq) * a.n_eff + pos] = key[qq];
                    continue;
                }
                const bool p = valid && (key[qq] < cthr[qq] || (key[qq] == cthr[qq] && pos <= cpos[qq]));
                const unsigned long long msk = __ballot(p);
                if (msk) {
                    const int w = ccount[qq] + __popcll(msk & ((1ull << lane) - 1ull));
                    if (p && w < a.cap) {
                        const int64_t at =
                            (((int64_t)(q0 + qq) * a.splits + split) * kPqWaves + wave) * a.cap + w;
                        a.cand_keys[at] = key[qq];
                        a.cand_pos[at] = (int)pos;
                    }
                    ccount[qq] += __popcll(msk);
                }
            }
        } else {
            // one test for the row's keys of all QPB queries (insertions are rare once the
            // lists have filled), then the queries that have a candidate
            bool any = false;
#pragma unroll
            for (int qq = 0; qq < QPB; ++qq) any |= key[qq] <= tau_k[qq] && qok[qq];
            if (!__ballot(valid && any)) return;
#pragma unroll
            for (int qq = 0; qq < QPB; ++qq) {
                unsigned long long msk = __ballot(valid && qok[qq] && key[qq] <= tau_k[qq]);
                while (msk) {
                    const int src = __builtin_ctzll(msk);
                    msk &= msk - 1;
                    const float ck = readlane_f(key[qq], src);
                    const int cid = base + src;
                    if (!cand_less(ck, cid, tau_k[qq], tau_i[qq])) continue;
                    list_insert<KP>(list_k(qq), list_i(qq), 0, a.kl, ck, cid, tau_k[qq],
                                    tau_i[qq]);
                }
            }
        }
    };

    // positions fit 32 bits (at most 2^31 - 2 rows; host-checked)
    const int row0 = (int)((int64_t)split * a.rows_per_split);
    const int row1 = (int)min(a.n_eff, (int64_t)row0 + a.rows_per_split);
    if constexpr (M > 0) {
        using CR = CodeRow<M>;
        using E = typename Entry<QPB>::type;
        // every load below is in bounds: positions past the split's end read its last row
        // (the host launches only non-empty splits), whose key is never used
        const int last = max(row1 - 1, row0);
        // (row ids are int32 until used, so that a row id's load is waited for only where
        // the next iteration reads its code row)
        auto row_of = [&](int pos) __attribute__((always_inline)) -> int {
            const int p = min(pos, last);
            const int r = a.rowidx ? a.rowidx[p] : (int)p;
            PX_DCHECK(a.dbg, kDbgPq, p < a.n_eff && r >= 0 && r < a.rows);
            return r;
        };
        auto code_of = [&](int row) __attribute__((always_inline)) {
            return *reinterpret_cast<const CR*>(a.codes + (int64_t)row * M);
        };
        // (a split's positions plus two steps stay below 2^31: splits end at n_eff)
        int base = row0 + wave * 64;
        CR cur = code_of(row_of(base + lane));
        int r_next = row_of(min(base + kPqThreads, last) + lane);
        for (; base < row1; base += kPqThreads) {
            const int pos = base + lane;
            const bool valid = pos < row1;
            // the next iteration's code row, and (filtered) the row id of the one after
            const CR nxt = code_of(r_next);
            r_next = row_of(min(base + 2 * kPqThreads, last) + lane);
            E e[M];
#pragma unroll
            for (int sub = 0; sub < M; ++sub)
                e[sub] = *reinterpret_cast<const E*>(lut + (sub * ks + cur.c[sub]) * QPB);
            float key[QPB];
#pragma unroll
            for (int qq = 0; qq < QPB; ++qq) key[qq] = 0.0f;
#pragma unroll
            for (int sub = 0; sub < M; ++sub) add_entry<QPB>(key, e[sub]);
            consume(base, pos, valid, key);
            cur = nxt;
        }
    } else {
        for (int base = row0 + wave * 64; base < row1; base += kPqThreads) {
            const int pos = base + lane;
            const bool valid = pos < row1;
            float key[QPB];
#pragma unroll
            for (int qq = 0; qq < QPB; ++qq) key[qq] = 0.0f;
            if (valid) {
                const int64_t row = a.rowidx ? (int64_t)a.rowidx[pos] : pos;
                PX_DCHECK(a.dbg, kDbgPq, pos < a.n_eff && row >= 0 && row < a.rows);
                const uint8_t* cp = a.codes + row * m;
                for (int sub = 0; sub < m; ++sub)
                    add_entry<QPB>(key, *reinterpret_cast<const typename Entry<QPB>::type*>(
                                            lut + (sub * ks + cp[sub]) * QPB));
            }
            consume(base, pos, valid, key);
        }
    }

    if constexpr (COLLECT) {
        if (!a.dense && lane == 0) {
#pragma unroll
            for (int qq = 0; qq < QPB; ++qq)
                if (qok[qq])
                    a.cand_count[((int64_t)(q0 + qq) * a.splits + split) * kPqWaves + wave] =
                        ccount[qq];
        }
        return;
    }
    // part[q][split * waves + wave][0..kl)
    const int width = a.splits * kPqWaves;
#pragma unroll
    for (int qq = 0; qq < QPB; ++qq) {
        if (q0 + qq >= a.nq) break;
        const int64_t off = ((int64_t)(q0 + qq) * width + split * kPqWaves + wave) * a.kl;
        for (int s = lane; s < a.kl; s += 64) {
            a.part_keys[off + s] = list_k(qq)[s];
            a.part_ids[off + s] = list_i(qq)[s];
        }
    }
}

// One launch of a PQ scan variant; dynamic LDS past 64 KB (lists of 32 or more beside the
// 64 KB of LUTs) is allowed for the kernel first, once per variant.
template <int QPB, int KP, int M, bool COLLECT, int KS = 0>
static hipError_t launch_one(const PqScanArgs& a, hipStream_t s) {
    const int64_t groups = (a.nq + QPB - 1) / QPB;
    const dim3 grid((unsigned)(groups * a.splits));
    const size_t lds = pq_lds_bytes(QPB, a.m, a.ks, KP);
    static size_t allowed = 65536;
    if (lds > allowed) {
        const hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(pq_scan_kernel<QPB, KP, M, COLLECT, KS>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        allowed = lds;
    }
    hipLaunchKernelGGL((pq_scan_kernel<QPB, KP, M, COLLECT, KS>), grid, dim3(kPqThreads), lds, s,
                       a);
    return hipGetLastError();
}

template <int QPB, int KP, bool COLLECT>
static hipError_t launch_pq_q(const PqScanArgs& a, hipStream_t s) {
    if (a.m == 16 && a.ks == 256) return launch_one<QPB, KP, 16, COLLECT, 256>(a, s);
    if (a.m == 16) return launch_one<QPB, KP, 16, COLLECT>(a, s);
    if (a.m == 8 && a.ks == 256) return launch_one<QPB, KP, 8, COLLECT, 256>(a, s);
    if (a.m == 8) return launch_one<QPB, KP, 8, COLLECT>(a, s);
    return launch_one<QPB, KP, 0, COLLECT>(a, s);
}

template <int KP>
static hipError_t launch_pq_k(const PqScanArgs& a, hipStream_t s) {
    switch (pq_queries_per_block(a.m, a.ks)) {
        case 4: return launch_pq_q<4, KP, false>(a, s);
        case 2: return launch_pq_q<2, KP, false>(a, s);
        default: return launch_pq_q<1, KP, false>(a, s);
    }
}

hipError_t launch_pq_collect(const PqScanArgs& a, hipStream_t s) {
    switch (pq_queries_per_block(a.m, a.ks)) {
        case 4: return launch_pq_q<4, 1, true>(a, s);
        case 2: return launch_pq_q<2, 1, true>(a, s);
        default: return launch_pq_q<1, 1, true>(a, s);
    }
}

hipError_t launch_pq_scan(const PqScanArgs& a, hipStream_t s) {
    switch (pq_list_capacity(a.kl)) {
        case 16: return launch_pq_k<16>(a, s);
        case 32: return launch_pq_k<32>(a, s);
        case 64: return launch_pq_k<64>(a, s);
        default: return launch_pq_k<128>(a, s);
    }
}

// ---- LDS read-rate calibration (the PQ scan's roofline) -----------------------------------
// Each thread reads 16-byte slots of a 64 KB table in LDS, sixteen a loop iteration as the
// ADC scan issues its gathers (immediate subtable offsets 4 KB apart): RANDOM = 0, slots
// (lane + 64 i) mod 256 of each subtable, so the 16 lanes of every quarter-wave read 16
// consecutive slots (no bank conflict); RANDOM = 1, one random byte (an LCG) per read, the
// ADC scan's pattern on uniform codes. Every slot is below 4096; each thread writes one sum.
namespace {
template <bool RANDOM>
__global__ __launch_bounds__(512) void lds_gather_kernel(float* out, int iters) {
    __shared__ __attribute__((aligned(16))) float4 tab[4096];
    const int tid = threadIdx.x, lane = tid & 63;
    for (int x = tid; x < 4096; x += 512) tab[x] = make_float4(x, x + 1, x + 2, x + 3);
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    unsigned h = (blockIdx.x * 512u + tid) * 2654435761u;
    for (int i = 0; i < iters; ++i) {
        unsigned c4[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            h = h * 1664525u + 1013904223u;
            c4[w] = h;
        }
        float4 v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int code = (int)((c4[u >> 2] >> (8 * (u & 3))) & 255u);
            v[u] = tab[u * 256 + (RANDOM ? code : ((lane + 64 * i) & 255))];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            acc.x = acc.x + v[u].x;
            acc.y = acc.y + v[u].y;
            acc.z = acc.z + v[u].z;
            acc.w = acc.w + v[u].w;
        }
    }
    out[blockIdx.x * 512 + tid] = acc.x + acc.y + acc.z + acc.w;
}
}  // namespace

int lds_gather_threads() { return 512; }

hipError_t launch_lds_gather(int random, int blocks, int iters, float* out, hipStream_t s) {
    if (random)
        hipLaunchKernelGGL(lds_gather_kernel<true>, dim3(blocks), dim3(512), 0, s, out, iters);
    else
        hipLaunchKernelGGL(lds_gather_kernel<false>, dim3(blocks), dim3(512), 0, s, out, iters);
    return hipGetLastError();
}

}  // namespace px
