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

constexpr int kPqWaves = 4;
constexpr int kPqThreads = kPqWaves * 64;

int pq_list_capacity(int kl) {
    if (kl <= 16) return 16;
    if (kl <= 32) return 32;
    if (kl <= 64) return 64;
    return 128;
}
int pq_lists_per_split() { return kPqWaves; }

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

// key[qq] += entry of query qq, for the QPB query-interleaved entries at e (one LDS read).
template <int QPB>
__device__ __forceinline__ void add_entries(float (&key)[QPB], const float* e) {
    if constexpr (QPB == 4) {
        const float4 v = *reinterpret_cast<const float4*>(e);
        key[0] = key[0] + v.x;
        key[1] = key[1] + v.y;
        key[2] = key[2] + v.z;
        key[3] = key[3] + v.w;
    } else if constexpr (QPB == 2) {
        const float2 v = *reinterpret_cast<const float2*>(e);
        key[0] = key[0] + v.x;
        key[1] = key[1] + v.y;
    } else {
        key[0] = key[0] + e[0];
    }
}

// M > 0: compile-time subspace count with a vector code load; M == 0: runtime m.
// COLLECT (k past the lists): no lists; each wave appends every row at or below its
// query's threshold (key, position) to its region of (query slot, split, wave), or, with
// a.dense, writes every key to cand_keys[q][n_eff].
template <int QPB, int KP, int M, bool COLLECT = false>
__global__ __launch_bounds__(kPqThreads) void pq_scan_kernel(PqScanArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lut[];  // [m * ks][QPB]
    __shared__ float lkeys[kPqWaves][QPB][KP];
    __shared__ int lids[kPqWaves][QPB][KP];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m = M > 0 ? M : a.m;
    const int lut_len = m * a.ks;
    const int qg = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
    const int q0 = qg * QPB;
    const float kInf = __int_as_float(0x7f800000);
    // query index of slot q0 + qq (a retry round lists the queries it serves)
    auto qidx = [&](int qq) { return (COLLECT && a.qlist) ? a.qlist[q0 + qq] : q0 + qq; };

    // lut[(sub * ks + c) * QPB + qq] = l2_sqr(q_sub, centroid) | -inner_product(q_sub, centroid)
    for (int x = tid; x < QPB * lut_len; x += kPqThreads) {
        const int qq = x % QPB;
        const int rest = x / QPB;
        const int sub = rest / a.ks;
        const int c = rest - sub * a.ks;
        float v = 0.f;
        if (q0 + qq < a.nq) {
            const float* qs = a.queries + (int64_t)qidx(qq) * a.dim + sub * a.dsub;
            const float* cen = a.codebooks + ((int64_t)sub * a.ks + c) * a.dsub;
            v = a.metric == 0 ? ref_l2_sqr(qs, cen, a.dsub) : -ref_inner_product(qs, cen, a.dsub);
        }
        lut[x] = v;
    }
    if constexpr (!COLLECT) {
        for (int x = lane; x < QPB * KP; x += 64) {
            lkeys[wave][x / KP][x % KP] = kInf;
            lids[wave][x / KP][x % KP] = kIdNone;
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

    const int64_t row0 = (int64_t)split * a.rows_per_split;
    const int64_t row1 = min(a.n_eff, row0 + a.rows_per_split);
    for (int64_t base = row0 + wave * 64; base < row1; base += kPqThreads) {
        const int64_t pos = base + lane;
        const bool valid = pos < row1;
        float key[QPB];
#pragma unroll
        for (int qq = 0; qq < QPB; ++qq) key[qq] = 0.0f;
        if (valid) {
            const int64_t row = a.rowidx ? (int64_t)a.rowidx[pos] : pos;
            PX_DCHECK(a.dbg, kDbgPq, pos < a.n_eff && row >= 0 && row < a.rows);
            if (M > 0) {
                const CodeRow<(M > 0 ? M : 1)> cr =
                    *reinterpret_cast<const CodeRow<(M > 0 ? M : 1)>*>(a.codes + row * M);
#pragma unroll
                for (int sub = 0; sub < (M > 0 ? M : 1); ++sub)
                    add_entries<QPB>(key, lut + (sub * a.ks + cr.c[sub]) * QPB);
            } else {
                const uint8_t* cp = a.codes + row * m;
                for (int sub = 0; sub < m; ++sub)
                    add_entries<QPB>(key, lut + (sub * a.ks + cp[sub]) * QPB);
            }
        }
        if constexpr (COLLECT) {
#pragma unroll
            for (int qq = 0; qq < QPB; ++qq) {
                if (a.dense) {
                    if (valid && qok[qq]) a.cand_keys[(int64_t)(q0 + qq) * a.n_eff + pos] = key[qq];
                    continue;
                }
                const bool p = valid && (key[qq] < cthr[qq] ||
                                         (key[qq] == cthr[qq] && pos <= (int64_t)cpos[qq]));
                const unsigned long long m = __ballot(p);
                if (m) {
                    const int w = ccount[qq] + __popcll(m & ((1ull << lane) - 1ull));
                    if (p && w < a.cap) {
                        const int64_t at =
                            (((int64_t)(q0 + qq) * a.splits + split) * kPqWaves + wave) * a.cap + w;
                        a.cand_keys[at] = key[qq];
                        a.cand_pos[at] = (int)pos;
                    }
                    ccount[qq] += __popcll(m);
                }
            }
            continue;
        }
#pragma unroll
        for (int qq = 0; qq < QPB; ++qq) {
            unsigned long long msk = __ballot(valid && qok[qq] && key[qq] <= tau_k[qq]);
            while (msk) {
                const int src = __builtin_ctzll(msk);
                msk &= msk - 1;
                const float ck = readlane_f(key[qq], src);
                const int cid = (int)(base + src);
                if (!cand_less(ck, cid, tau_k[qq], tau_i[qq])) continue;
                list_insert<KP>(&lkeys[wave][qq][0], &lids[wave][qq][0], 0, a.kl, ck, cid,
                                tau_k[qq], tau_i[qq]);
            }
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
            a.part_keys[off + s] = lkeys[wave][qq][s];
            a.part_ids[off + s] = lids[wave][qq][s];
        }
    }
}

template <int QPB, int KP>
static hipError_t launch_pq_q(const PqScanArgs& a, hipStream_t s) {
    const int64_t groups = (a.nq + QPB - 1) / QPB;
    const dim3 grid((unsigned)(groups * a.splits));
    const size_t lds = (size_t)QPB * a.m * a.ks * sizeof(float);
    if (a.m == 16)
        hipLaunchKernelGGL((pq_scan_kernel<QPB, KP, 16>), grid, dim3(kPqThreads), lds, s, a);
    else if (a.m == 8)
        hipLaunchKernelGGL((pq_scan_kernel<QPB, KP, 8>), grid, dim3(kPqThreads), lds, s, a);
    else
        hipLaunchKernelGGL((pq_scan_kernel<QPB, KP, 0>), grid, dim3(kPqThreads), lds, s, a);
    return hipGetLastError();
}

template <int KP>
static hipError_t launch_pq_k(const PqScanArgs& a, hipStream_t s) {
    switch (pq_queries_per_block(a.m, a.ks)) {
        case 4: return launch_pq_q<4, KP>(a, s);
        case 2: return launch_pq_q<2, KP>(a, s);
        default: return launch_pq_q<1, KP>(a, s);
    }
}

template <int QPB>
static hipError_t launch_pq_collect_q(const PqScanArgs& a, hipStream_t s) {
    const int64_t groups = (a.nq + QPB - 1) / QPB;
    const dim3 grid((unsigned)(groups * a.splits));
    const size_t lds = (size_t)QPB * a.m * a.ks * sizeof(float);
    if (a.m == 16)
        hipLaunchKernelGGL((pq_scan_kernel<QPB, 1, 16, true>), grid, dim3(kPqThreads), lds, s, a);
    else if (a.m == 8)
        hipLaunchKernelGGL((pq_scan_kernel<QPB, 1, 8, true>), grid, dim3(kPqThreads), lds, s, a);
    else
        hipLaunchKernelGGL((pq_scan_kernel<QPB, 1, 0, true>), grid, dim3(kPqThreads), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_pq_collect(const PqScanArgs& a, hipStream_t s) {
    switch (pq_queries_per_block(a.m, a.ks)) {
        case 4: return launch_pq_collect_q<4>(a, s);
        case 2: return launch_pq_collect_q<2>(a, s);
        default: return launch_pq_collect_q<1>(a, s);
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

}  // namespace px
