// px_index.hip -- host side of libproxima_px.so: FlatIndex / PqIndex handles and the C ABI.
//
// Mirrors the reference's core API (crates/core/src/flat.rs, pq.rs) and its GPU seam
// (crates/core/src/gpu.rs:10-15, crates/core/cuda/knn.cu:123-180). Rows are appended on
// the host and mirrored into HBM (row-major, dims padded to a multiple of 8, squared
// norms alongside); searches run entirely on the GPU. There is no CPU search path: with
// no gfx950 device a search fails with PX_ERR_DEVICE.
#include "proxima_px.h"
#include "px_host.h"
#include "px_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define PX_HIP(expr)                                                                        \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return fail((int)e_, std::string(#expr) + " failed: " + hipGetErrorString(e_)); \
    } while (0)

// Host-side index checks of the launch geometry (cheap, always on): a failure is a bug in
// this library, reported as PX_ERR_ARG naming the condition and line, before any launch.
#define PX_INTERNAL(cond)                                                                   \
    do {                                                                                    \
        if (!(cond))                                                                        \
            return fail(PX_ERR_ARG, std::string("internal check failed: ") + #cond +        \
                                        " (px_index.hip:" + std::to_string(__LINE__) + ")"); \
    } while (0)

#define PX_TRY(expr)             \
    do {                         \
        int rc_ = (expr);        \
        if (rc_ != PX_OK) return rc_; \
    } while (0)

// all_finite, and in the same pass whether every value is exactly an fp16 zero or normal
// number (*f16_exact): zero, or a magnitude in [2^-14, 2^16) with the 13 low mantissa bits
// clear -- what to_f16_kernel checks on the device. About 2.5 times all_finite's cost, so
// used on small batches only (where it spares a device read-back that costs more).
bool finite_and_f16(const float* x, int64_t len, bool* f16_exact) {
    constexpr int64_t kBlock = 4096;
    uint32_t inexact = 0;
    for (int64_t b = 0; b < len; b += kBlock) {
        const int64_t e = std::min(len, b + kBlock);
        uint32_t bad = 0, inx = 0;
        for (int64_t i = b; i < e; ++i) {
            uint32_t u;
            std::memcpy(&u, x + i, sizeof(u));
            const uint32_t a = u & 0x7fffffffu;
            bad |= (uint32_t)(a >= 0x7f800000u);
            inx |= (uint32_t)(a != 0) &
                   ((uint32_t)(a - 0x38800000u >= 0x0f000000u) | (uint32_t)((a & 0x1fffu) != 0));
        }
        if (bad) return false;
        inexact |= inx;
    }
    *f16_exact = inexact == 0;
    return true;
}

bool all_finite(const float* x, int64_t len) {
    // blocks of 4,096 values, the exponent bits of each compared and OR-ed with no early
    // exit inside a block, so that the loop vectorizes (a value is NaN or infinite exactly
    // when its exponent bits are all ones)
    constexpr int64_t kBlock = 4096;
    for (int64_t b = 0; b < len; b += kBlock) {
        const int64_t e = std::min(len, b + kBlock);
        uint32_t bad = 0;
        for (int64_t i = b; i < e; ++i) {
            uint32_t u;
            std::memcpy(&u, x + i, sizeof(u));
            bad |= (uint32_t)((u & 0x7f800000u) == 0x7f800000u);
        }
        if (bad) return false;
    }
    return true;
}

// The library's own device allocations (not the caller's px_dev_* buffers, nor the static
// array of the no-allocation entry point) go through dev_malloc / dev_free, which keep
// their total. PX_DEVICE_BUDGET (bytes, read at every allocation) caps it: an allocation
// that would pass the cap fails with hipErrorOutOfMemory, as on a full device -- how the
// out-of-memory paths are tested.
std::mutex g_alloc_mu;
std::unordered_map<void*, size_t> g_alloc_sizes;
int64_t g_alloc_total = 0;

hipError_t dev_malloc(void** p, size_t bytes) {
    *p = nullptr;
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    if (const char* e = std::getenv("PX_DEVICE_BUDGET")) {
        char* end = nullptr;
        const long long budget = std::strtoll(e, &end, 10);
        if (end != e && g_alloc_total + (int64_t)bytes > budget) return hipErrorOutOfMemory;
    }
    const hipError_t r = hipMalloc(p, bytes);
    if (r == hipSuccess) {
        g_alloc_sizes[*p] = bytes;
        g_alloc_total += (int64_t)bytes;
    }
    return r;
}

void dev_free(void* p) {
    if (!p) return;
    (void)hipFree(p);
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    const auto it = g_alloc_sizes.find(p);
    if (it != g_alloc_sizes.end()) {
        g_alloc_total -= (int64_t)it->second;
        g_alloc_sizes.erase(it);
    }
}

template <class T>
hipError_t dev_malloc(T** p, size_t bytes) {
    void* v = nullptr;
    const hipError_t r = dev_malloc(&v, bytes);
    *p = static_cast<T*>(v);
    return r;
}

// Grow-only device buffer.
struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    int reserve(size_t bytes) {
        if (bytes <= cap) return PX_OK;
        dev_free(p);
        p = nullptr;
        cap = 0;
        const size_t want = std::max<size_t>(bytes, 256);
        PX_HIP(dev_malloc(&p, want));
        cap = want;
        return PX_OK;
    }
    void release() {
        dev_free(p);
        p = nullptr;
        cap = 0;
    }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};

struct DeviceInfo {
    int device = -1;
    int cus = 0;
};

// Binds the calling thread to the library's device (the one current when the first
// handle bound it) and checks it is a gfx950.
int bind_device(DeviceInfo& info) {
    if (info.device >= 0) {
        PX_HIP(hipSetDevice(info.device));
        return PX_OK;
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(PX_ERR_DEVICE, "no HIP device is visible: proxima_amd searches run only on a "
                                   "gfx950 (MI355X) GPU and have no CPU path");
    int dev = 0;
    PX_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    PX_HIP(hipGetDeviceProperties(&prop, dev));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(PX_ERR_DEVICE, std::string("device ") + std::to_string(dev) + " is " +
                                       prop.gcnArchName + "; libproxima_px.so is built for gfx950");
    info.device = dev;
    info.cus = prop.multiProcessorCount;
    return PX_OK;
}

struct Timing {
    bool enabled = false;
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    float scan_ms = 0.f, total_ms = 0.f;
    int splits = 0, blocks = 0;
    int ensure() {
        if (!enabled) return PX_OK;
        for (auto& e : ev)
            if (!e) PX_HIP(hipEventCreate(&e));
        return PX_OK;
    }
    void destroy() {
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
    }
};

// Scratch shared by both index kinds for one search.
struct Workspace {
    DevBuf q, qn, mask, rowidx, scratch, count, part_k, part_i, out_ids, out_d, gtau, gbest;
    // collect path (k' past the lists)
    DevBuf thr_k, thr_p, lad_k, lad_p, rung, status, cand_k, cand_p, cand_n, samp_row, qlist;
    DevBuf cand_d;           // smallest dropped key of each overflowing region
    DevBuf qh;               // a batch's queries as fp16 (the fp16 scans; px_flat::d_xh)
    DevBuf fflag;            // finiteness verdicts of list-path searches (next_finite_seq)
    DevBuf spinw;            // the list scans' stage-sync give-up word (FlatScanArgs::spin_fail)
    int fseq = 0;
    DevBuf dbgw;             // debug build: the debug word of the kernels' index checks ...
    int* dbg = nullptr;      // ... while a search runs (null in the product build)
    DevBuf qraw;             // host-path queries before padding to dp
    DevBuf sort_scratch;     // k past PX_MAX_K: sort keys, positions, radix-sort storage
    // Read-backs of the search path (pinned, mapped, coherent): written by a kernel
    // (launch_copy_to_host) through their device addresses *_dev, read by the host after
    // the stream drains
    int* h_count = nullptr;      // two ints (one read-back, or a merge's two verdicts)
    int* h_count_dev = nullptr;
    int* h_status = nullptr;     // h_status_cap ints
    int* h_status_dev = nullptr;
    int64_t h_status_cap = 0;
    // pinned staging for the host-buffer entry points: queries in, results out (pageable
    // copies are staged by the runtime, and 2-D ones row by row)
    char* h_in = nullptr;
    char* h_out = nullptr;
    size_t h_in_cap = 0, h_out_cap = 0;
    static int ensure_host(char*& buf, size_t& cap, size_t bytes) {
        if (bytes <= cap) return PX_OK;
        if (buf) (void)hipHostFree(buf);
        buf = nullptr;
        cap = 0;
        const size_t want = std::max<size_t>(bytes, 4096);
        PX_HIP(hipHostMalloc(reinterpret_cast<void**>(&buf), want));
        cap = want;
        return PX_OK;
    }
    static int mapped_ints(int** host, int** dev, int64_t n) {
        PX_HIP(hipHostMalloc(reinterpret_cast<void**>(host), sizeof(int) * std::max<int64_t>(n, 1),
                             hipHostMallocMapped | hipHostMallocCoherent));
        const hipError_t e = hipHostGetDevicePointer(reinterpret_cast<void**>(dev), *host, 0);
        if (e != hipSuccess) {
            (void)hipHostFree(*host);
            *host = *dev = nullptr;
            PX_HIP(e);
        }
        return PX_OK;
    }
    int ensure_pinned() {
        if (!h_count) PX_TRY(mapped_ints(&h_count, &h_count_dev, 2));
        return PX_OK;
    }
    int ensure_status(int64_t n) {
        if (n <= h_status_cap) return PX_OK;
        if (h_status) (void)hipHostFree(h_status);
        h_status = h_status_dev = nullptr;
        h_status_cap = 0;
        PX_TRY(mapped_ints(&h_status, &h_status_dev, n));
        h_status_cap = n;
        return PX_OK;
    }
    void release() {
        for (DevBuf* b : {&q, &qn, &mask, &rowidx, &scratch, &count, &part_k, &part_i, &out_ids,
                          &out_d, &gtau, &gbest, &thr_k, &thr_p, &lad_k, &lad_p, &rung, &status,
                          &cand_k, &cand_p, &cand_n, &cand_d, &qh, &samp_row, &qlist,
                          &sort_scratch,
                          &fflag, &spinw,
                          &dbgw})
            b->release();
        fseq = 0;
        if (h_count) (void)hipHostFree(h_count);
        h_count = h_count_dev = nullptr;
        if (h_status) (void)hipHostFree(h_status);
        h_status = h_status_dev = nullptr;
        h_status_cap = 0;
        qraw.release();
        if (h_in) (void)hipHostFree(h_in);
        if (h_out) (void)hipHostFree(h_out);
        h_in = h_out = nullptr;
        h_in_cap = h_out_cap = 0;
    }
};

// Host queries [nq][dim] to device [nq][dp] (zero pad columns) through pinned staging.
int upload_queries(Workspace& ws, const float* queries, int64_t nq, int64_t dim, int64_t dp,
                   hipStream_t s, const float** d_q) {
    const size_t bytes = sizeof(float) * (size_t)(nq * dim);
    PX_TRY(Workspace::ensure_host(ws.h_in, ws.h_in_cap, bytes));
    PX_TRY(ws.q.reserve(sizeof(float) * nq * dp));
    if (dp != dim) PX_TRY(ws.qraw.reserve(bytes));
    char* dst = static_cast<char*>(dp == dim ? ws.q.p : ws.qraw.p);
    // staged in 1 MB pieces: the copy engine moves one while the host stages the next
    constexpr size_t kPiece = (size_t)1 << 20;
    for (size_t off = 0; off < bytes; off += kPiece) {
        const size_t n = std::min(kPiece, bytes - off);
        std::memcpy(ws.h_in + off, reinterpret_cast<const char*>(queries) + off, n);
        PX_HIP(hipMemcpyAsync(dst + off, ws.h_in + off, n, hipMemcpyHostToDevice, s));
    }
    if (dp != dim)
        PX_HIP(px::launch_pad_rows(ws.qraw.as<float>(), nq, (int)dim, (int)dp, ws.q.as<float>(), s));
    *d_q = ws.q.as<float>();
    return PX_OK;
}

// Device results [nq][k] to the caller's host buffers through pinned staging; waits.
int download_results(Workspace& ws, int64_t nq, int64_t k, hipStream_t s, int64_t* out_ids,
                     float* out_d) {
    const size_t bi = sizeof(int64_t) * (size_t)(nq * k), bd = sizeof(float) * (size_t)(nq * k);
    PX_TRY(Workspace::ensure_host(ws.h_out, ws.h_out_cap, bi + bd));
    PX_HIP(hipMemcpyAsync(ws.h_out, ws.out_ids.p, bi, hipMemcpyDeviceToHost, s));
    PX_HIP(hipMemcpyAsync(ws.h_out + bi, ws.out_d.p, bd, hipMemcpyDeviceToHost, s));
    PX_HIP(hipStreamSynchronize(s));
    std::memcpy(out_ids, ws.h_out, bi);
    std::memcpy(out_d, ws.h_out + bi, bd);
    return PX_OK;
}

// One device int read back into h: by a kernel when h is mapped pinned memory (h_dev its
// device address), else (the caller's own memory) by a copy. Waits for the stream.
int read_back_int(const int* d, int* h, int* h_dev, hipStream_t s) {
    if (h_dev) PX_HIP(px::launch_copy_to_host(d, h_dev, 1, s));
    else PX_HIP(hipMemcpyAsync(h, d, sizeof(int), hipMemcpyDeviceToHost, s));
    PX_HIP(hipStreamSynchronize(s));
    return PX_OK;
}

// Compacts a device keep-mask of n rows into ascending row ids (rowidx, n ints; cscr,
// mask_compact_scratch(n) ints; d_count one int) and reads the kept count back through
// h_count (read_back_int); returns it in *n_eff.
int compact_mask_into(const uint8_t* d_mask, int64_t n, int* rowidx, int* cscr, int* d_count,
                      int* h_count, int* h_count_dev, hipStream_t s, int64_t* n_eff) {
    PX_HIP(px::launch_mask_compact(d_mask, n, rowidx, cscr, d_count, s));
    PX_TRY(read_back_int(d_count, h_count, h_count_dev, s));
    *n_eff = *h_count;
    return PX_OK;
}

int compact_mask(Workspace& ws, const uint8_t* d_mask, int64_t n, hipStream_t s, int64_t* n_eff,
                 const int** rowidx) {
    PX_TRY(ws.rowidx.reserve(sizeof(int) * std::max<int64_t>(n, 1)));
    PX_TRY(ws.scratch.reserve(sizeof(int) * px::mask_compact_scratch(n)));
    PX_TRY(ws.count.reserve(sizeof(int)));
    PX_TRY(ws.ensure_pinned());
    PX_TRY(compact_mask_into(d_mask, n, ws.rowidx.as<int>(), ws.scratch.as<int>(),
                             ws.count.as<int>(), ws.h_count, ws.h_count_dev, s, n_eff));
    *rowidx = ws.rowidx.as<int>();
    return PX_OK;
}

// Device queries (count floats) must be finite, as flat.rs:114-117 asserts of every query:
// checked on the device (d_flag, one int), and the host waits for the answer (read through
// h_flag, read_back_int) before any search kernel runs.
int check_finite_into(const float* d_x, int64_t count, int* d_flag, int* h_flag, int* h_flag_dev,
                      hipStream_t s) {
    PX_HIP(px::launch_nonfinite_check(d_x, count, d_flag, s));
    PX_TRY(read_back_int(d_flag, h_flag, h_flag_dev, s));
    if (*h_flag)
        return fail(PX_ERR_NONFINITE, "query must not contain NaN or infinite values");
    return PX_OK;
}

int nonfinite_error() {
    return fail(PX_ERR_NONFINITE, "query must not contain NaN or infinite values");
}

// The device queries of a search whose finiteness check has not run yet (x: count floats).
// The per-split list path checks them in its first kernel, hands the verdict to its scan
// and merge (which do nothing for a failed search) and reads it back with its last wait;
// every other path checks them first (check_device_finite).
struct PendingCheck {
    const float* x;
    int64_t count;
};

// The sequence number of a list-path search's finiteness check: its flag (ws.fflag) holds
// the largest number of a search that failed, so no search clears it. Cleared on first use
// and when the numbers wrap.
int next_finite_seq(Workspace& ws, hipStream_t s, int* seq) {
    PX_TRY(ws.fflag.reserve(sizeof(int)));
    PX_TRY(ws.ensure_pinned());
    if (ws.fseq <= 0 || ws.fseq == INT_MAX) {
        PX_HIP(px::launch_fill_int(ws.fflag.as<int>(), 1, 0, s));
        ws.fseq = 0;
    }
    *seq = ++ws.fseq;
    return PX_OK;
}

#ifdef PX_DEBUG
constexpr bool kDebugBuild = true;
#else
constexpr bool kDebugBuild = false;
#endif

// Debug build (-DPX_DEBUG): a search runs between debug_begin, which clears the debug word
// that the kernels' index checks (PX_DCHECK) record a failure in, and debug_end, which
// reads it and fails the search with PX_ERR_ARG naming the check's file and line.
int debug_begin(Workspace& ws, hipStream_t s) {
    if (!kDebugBuild) return PX_OK;
    PX_TRY(ws.dbgw.reserve(sizeof(int)));
    PX_TRY(ws.ensure_pinned());
    PX_HIP(px::launch_fill_int(ws.dbgw.as<int>(), 1, 0, s));
    ws.dbg = ws.dbgw.as<int>();
    return PX_OK;
}

int read_back_int(const int* d, int* h, int* h_dev, hipStream_t s);

int debug_end(Workspace& ws, hipStream_t s, int rc) {
    if (!kDebugBuild || !ws.dbg) return rc;
    int* d = ws.dbg;
    ws.dbg = nullptr;
    if (rc != PX_OK) return rc;
    PX_TRY(read_back_int(d, ws.h_count, ws.h_count_dev, s));
    const int v = *ws.h_count;
    if (v == 0) return PX_OK;
    static const char* const files[] = {"?", "px_flat.hip", "px_collect.hip", "px_pq.hip"};
    const int fid = v / 100000;
    return fail(PX_ERR_ARG, std::string("device index check failed at ") +
                                files[fid >= 1 && fid <= 3 ? fid : 0] + ":" +
                                std::to_string(v % 100000));
}

// Rows of several 128-dim chunks scanned over several rounds of workgroups take the
// XCD-major block order (FlatScanArgs::xcd_major); qpb: query slots per workgroup.
int xcd_major_for(const px::FlatScanArgs& a, int64_t qpb, int cus) {
    const int64_t blocks = (a.nq + qpb - 1) / qpb * (int64_t)a.splits;
    return a.dp > 128 && blocks > cus ? 1 : 0;
}

int check_device_finite(Workspace& ws, const float* d_x, int64_t count, hipStream_t s) {
    PX_TRY(ws.count.reserve(sizeof(int)));
    PX_TRY(ws.ensure_pinned());
    return check_finite_into(d_x, count, ws.count.as<int>(), ws.h_count, ws.h_count_dev, s);
}

// Number of corpus splits: enough workgroups to fill the GPU several times over, each
// split at least min_rows long, and at most kMaxMerge candidates per query to merge.
int choose_splits(int64_t n_eff, int64_t groups, int lists_per_split, int kl, int cus,
                  int64_t min_rows) {
    const int64_t target = 8LL * std::max(cus, 1);
    int64_t s = (target + groups - 1) / std::max<int64_t>(groups, 1);
    s = std::min<int64_t>(s, std::max<int64_t>(1, n_eff / std::max<int64_t>(min_rows, 1)));
    s = std::min<int64_t>(s, px::kMaxMerge / std::max(1, lists_per_split * kl));
    if (s >= 8) s = s / 8 * 8;  // consecutive blocks share a query tile; 8 XCDs
    return (int)std::max<int64_t>(s, 1);
}

// Corpus splits for the flat scan. Splits keep at least 256 rows, fit the merge
// (splits * kl <= kMaxMerge) and, for lists with 16-bit positions, at most
// kMaxNarrowSplitRows rows; a split count s gives rps = ceil(n_eff / s) rounded up to a
// whole tile and ceil(n_eff / rps) splits, as the callers compute them.
//  - Small lists (kl <= 32) and the collect scans: a workgroup holds a whole CU (its LDS
//    and registers allow one per CU), so a grid of B workgroups runs in ceil(B / cus)
//    rounds, each about as long as one split: rps rows plus about one tile of fixed cost
//    (query loads, the first tile's sort, the write-back). The count minimising
//    rounds * (rps + 64) is taken; among counts within 1% of that minimum, the one giving
//    the most rounds up to four (later rounds even out workgroups that finish at
//    different times), then a multiple of 8 (each XCD then sees a fixed subset of splits
//    across query tiles), then the fewest splits (less to merge).
//  - Large lists: every split builds its own list, and insertions grow with splits x kl,
//    so the smallest count giving one round at 90% occupancy.
int choose_flat_splits(int64_t n_eff, int64_t groups, int kl, int cus, bool narrow_ids) {
    cus = std::max(cus, 1);
    const int64_t min_s =
        narrow_ids ? std::max<int64_t>(1, (n_eff + px::kMaxNarrowSplitRows - 1) /
                                              px::kMaxNarrowSplitRows)
                   : 1;
    const int64_t max_s = std::max<int64_t>(
        min_s, std::min<int64_t>(n_eff / 256, px::kMaxMerge / std::max(kl, 1)));
    const int64_t top = std::max<int64_t>(min_s, std::min<int64_t>(max_s, 512));
    auto shape = [&](int64_t s, int64_t* rps, int64_t* splits) {
        int64_t r = (n_eff + s - 1) / s;
        r = std::max<int64_t>((r + 63) / 64 * 64, 64);
        if (narrow_ids) r = std::min<int64_t>(r, px::kMaxNarrowSplitRows);
        *rps = r;
        *splits = std::max<int64_t>(1, (n_eff + r - 1) / r);
    };
    if (kl > 32) {
        int64_t best = min_s;
        double best_eff = -1.0;
        for (int64_t s = 1; s <= top; s = s < 8 ? s * 2 : s + 8) {
            if (s < min_s) continue;
            const int64_t blocks = groups * s;
            const double eff = (double)blocks / (double)(((blocks + cus - 1) / cus) * cus);
            if (eff >= 0.90) return (int)s;
            if (eff > best_eff + 1e-9) {
                best = s;
                best_eff = eff;
            }
        }
        return (int)std::max<int64_t>(best, min_s);
    }
    double min_cost = 0.0;
    for (int64_t s = min_s; s <= top; ++s) {
        int64_t rps, splits;
        shape(s, &rps, &splits);
        const double cost = (double)((groups * splits + cus - 1) / cus) * (double)(rps + 64);
        if (s == min_s || cost < min_cost) min_cost = cost;
    }
    int64_t best = min_s, best_rounds = -1, best_splits = 0;
    bool best_m8 = false;
    for (int64_t s = min_s; s <= top; ++s) {
        int64_t rps, splits;
        shape(s, &rps, &splits);
        const int64_t rounds = (groups * splits + cus - 1) / cus;
        if ((double)rounds * (double)(rps + 64) > 1.01 * min_cost) continue;
        const int64_t r4 = std::min<int64_t>(rounds, 4);
        const bool m8 = splits % 8 == 0;
        if (r4 > best_rounds || (r4 == best_rounds && m8 && !best_m8) ||
            (r4 == best_rounds && m8 == best_m8 && splits < best_splits)) {
            best = s;
            best_rounds = r4;
            best_m8 = m8;
            best_splits = splits;
        }
    }
    return (int)best;
}

}  // namespace

// ---------------------------------------------------------------------------------------
// Handles
// ---------------------------------------------------------------------------------------
struct px_flat {
    int metric = 0;
    int smetric = 0;               // metric of the search in progress (set under mu): the
                                   // index's own, or the one knn_gpu_search names per call
    int64_t dim = 0, dp = 0;
    int64_t n = 0;                 // rows held (device + pending)
    std::vector<float> pending;    // rows not yet mirrored, [rows][dim]
    DeviceInfo dev;
    hipStream_t stream = nullptr;
    float* d_x = nullptr;          // [cap][dp]
    float* d_norm = nullptr;       // [cap]
    int64_t d_rows = 0, d_cap = 0;
    // 128-dim rows: their fp16 mirror [cap][128], kept while every value mirrored so far is
    // exactly an fp16 zero or normal number (integer descriptors such as SIFT's are). The
    // collect and list scans multiply in fp16 for a batch whose queries are exact too; the
    // vector-ALU scan of a few queries reads it widened. Dropped for good at the first row
    // that is not exact (or if its memory cannot be had).
    unsigned short* d_xh = nullptr;
    bool xh_exact = true;
    bool scan_f16 = true;          // px_flat_set_scan_f16
    int spin_limit = 0;            // stage-sync polls before a give-up, 0: the kernels' own
                                   // (px_flat_set_spin_limit; FlatScanArgs::spin_limit)
    bool last_f16 = false;         // the last search read d_xh (px_flat_last_scan_f16)
    int q_f16 = -1;                // host-array search in progress: its queries are exact in
                                   // fp16 (1) or not (0), checked on the host (batches of at
                                   // most 65,536 values); -1: unknown
    Workspace ws;
    Timing timing;
    int last_path = PX_PATH_LISTS; // selection path of the last search
    int last_rounds = 0;           // collect rounds of the last search (0: list path)
    std::mutex mu;
};

struct px_pq {
    int metric = 0;
    int64_t dim = 0, m = 0, nbits = 0, ks = 0, dsub = 0;
    bool trained = false;
    std::vector<float> codebooks;  // [m][ks][dsub]
    std::vector<uint8_t> codes;    // host copy of every code row, [n][m]
    int64_t n = 0;
    DeviceInfo dev;
    hipStream_t stream = nullptr;
    float* d_books = nullptr;
    bool books_on_device = false;
    uint8_t* d_codes = nullptr;
    int64_t d_rows = 0, d_cap = 0;
    Workspace ws;
    Timing timing;
    int last_rounds = 0;           // collect rounds of the last search (0: list path)
    std::mutex mu;
};

struct PxGpuIndex {
    px_flat* flat = nullptr;  // one corpus mirror (rows and squared norms) for both metrics
};

namespace {

int flat_bind(px_flat* f) {
    PX_TRY(bind_device(f->dev));
    if (!f->stream) PX_HIP(hipStreamCreateWithFlags(&f->stream, hipStreamNonBlocking));
    return PX_OK;
}

// Mirror pending rows into HBM: grow (doubling) if needed, upload with padding, norms.
int flat_sync(px_flat* f) {
    const int64_t add = (int64_t)(f->pending.size() / f->dim);
    if (add == 0) return PX_OK;
    PX_TRY(flat_bind(f));
    const int64_t need = f->d_rows + add;
    if (need > f->d_cap) {
        const int64_t cap = std::max<int64_t>({need, f->d_cap * 2, 1024});
        // the new buffers, freed on every early return below (the index keeps its old ones)
        // unless they have been adopted
        struct Fresh {
            float* x = nullptr;
            float* n = nullptr;
            unsigned short* h = nullptr;
            ~Fresh() {
                dev_free(x);
                dev_free(n);
                dev_free(h);
            }
        } fresh;
        float*& nx = fresh.x;
        float*& nn = fresh.n;
        PX_HIP(dev_malloc(&nx, sizeof(float) * cap * f->dp));
        if (dev_malloc(&nn, sizeof(float) * cap) != hipSuccess)
            return fail(hipErrorOutOfMemory, "device allocation of the corpus norms failed");
        if (f->d_rows) {
            PX_HIP(hipMemcpyAsync(nx, f->d_x, sizeof(float) * f->d_rows * f->dp,
                                  hipMemcpyDeviceToDevice, f->stream));
            PX_HIP(hipMemcpyAsync(nn, f->d_norm, sizeof(float) * f->d_rows,
                                  hipMemcpyDeviceToDevice, f->stream));
        }
        // the fp16 mirror grows with them, or is dropped if its memory cannot be had
        unsigned short*& nxh = fresh.h;
        if (f->dp == 128 && f->xh_exact) {
            if (dev_malloc(&nxh, sizeof(unsigned short) * cap * 128) != hipSuccess) {
                (void)hipGetLastError();
                nxh = nullptr;
                f->xh_exact = false;
            } else if (f->d_rows) {
                PX_HIP(hipMemcpyAsync(nxh, f->d_xh, sizeof(unsigned short) * f->d_rows * 128,
                                      hipMemcpyDeviceToDevice, f->stream));
            }
        }
        PX_HIP(hipStreamSynchronize(f->stream));
        dev_free(f->d_x);
        dev_free(f->d_norm);
        dev_free(f->d_xh);
        f->d_x = nx;
        f->d_norm = nn;
        f->d_xh = nxh;
        f->d_cap = cap;
        fresh.x = fresh.n = nullptr;  // adopted
        fresh.h = nullptr;
    }
    float* dst = f->d_x + f->d_rows * f->dp;
    if (f->dp == f->dim) {
        PX_HIP(hipMemcpyAsync(dst, f->pending.data(), sizeof(float) * add * f->dim,
                              hipMemcpyHostToDevice, f->stream));
    } else {
        // rows go up contiguously (a pitched host copy is staged row by row) in chunks of
        // 64 MB, and are padded to dp on the device
        const int64_t chunk =
            std::max<int64_t>(1, ((int64_t)64 << 20) / ((int64_t)sizeof(float) * f->dim));
        PX_TRY(f->ws.qraw.reserve(sizeof(float) * std::min(add, chunk) * f->dim));
        for (int64_t r = 0; r < add; r += chunk) {
            const int64_t nr = std::min(chunk, add - r);
            PX_HIP(hipMemcpyAsync(f->ws.qraw.p, f->pending.data() + r * f->dim,
                                  sizeof(float) * nr * f->dim, hipMemcpyHostToDevice, f->stream));
            PX_HIP(px::launch_pad_rows(f->ws.qraw.as<float>(), nr, (int)f->dim, (int)f->dp,
                                       dst + r * f->dp, f->stream));
        }
    }
    PX_HIP(px::launch_row_norms(dst, add, (int)f->dp, f->d_norm + f->d_rows, f->stream));
    int* xflag = nullptr;  // set if a new row is not exact in fp16
    if (f->d_xh) {
        PX_TRY(f->ws.count.reserve(sizeof(int)));
        PX_TRY(f->ws.ensure_pinned());
        xflag = f->ws.count.as<int>();
        PX_HIP(px::launch_fill_int(xflag, 1, 0, f->stream));
        PX_HIP(px::launch_to_f16(dst, add * 128, f->d_xh + f->d_rows * 128, xflag, f->stream));
    }
    PX_HIP(hipStreamSynchronize(f->stream));
    if (xflag) {
        PX_TRY(read_back_int(xflag, f->ws.h_count, f->ws.h_count_dev, f->stream));
        if (*f->ws.h_count) {
            dev_free(f->d_xh);
            f->d_xh = nullptr;
            f->xh_exact = false;
        }
    }
    f->d_rows = need;
    std::vector<float>().swap(f->pending);
    return PX_OK;
}

// Smallest k served by the threshold-collect path for batches of at least
// kCollectMinQueries queries. Below it the per-split lists are faster than a collect round
// that samples its thresholds (1M x 128, 10,000 queries: 23.6 ms a batch at k = 10 against
// 24.4); from k = 16 the collect path is ahead (24.8 / 23.7 ms at k = 16, 27.9 / 24.5 at
// k = 24, 46.5 / 25.9 at k = 64). Smaller k also goes to the collect path where its first
// round needs no sample (collect_bound_only). Smaller batches keep the lists, which need no
// sample pass and no host round trip. The PX_FLAT_COLLECT_FROM_K environment variable
// overrides the k (read once).
constexpr int64_t kCollectMinQueries = 256;
// Fewest rows on which the per-split list path takes the fp16 scan (its exactness check
// costs one read-back of the stream).
constexpr int64_t kF16ListMinRows = 65536;
int64_t collect_from_k() {
    static const int64_t v = [] {
        const char* e = std::getenv("PX_FLAT_COLLECT_FROM_K");
        return e && *e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)16;
    }();
    return v;
}

// Candidates beyond k whose keys are recomputed in the reference's arithmetic before the
// final order is taken (the MFMA keys differ from it by rounding).
constexpr int64_t kReRankMargin = 8;

// Splits and list layout of a fused list scan over n_eff rows with lists of kl.
struct ListPlan {
    int splits = 1;
    int64_t rps = 64, groups = 1;
};
// max_splits (>= 1) caps the split count (the no-allocation entry point's fixed scratch).
int plan_list_scan(int64_t n_eff, int64_t nq, int kl, int64_t dp, int cus, ListPlan* out,
                   int64_t k, int64_t max_splits = INT32_MAX) {
    const int kp = px::flat_list_capacity(kl);
    const int64_t qpb = px::flat_list_queries_per_block(kp, dp);
    const int64_t groups = (nq + qpb - 1) / qpb;
    const bool narrow = px::flat_list_narrow_ids(kp);
    int splits = (int)std::min<int64_t>(choose_flat_splits(n_eff, groups, kl, cus, narrow),
                                        std::max<int64_t>(1, max_splits));
    int64_t rps = (n_eff + splits - 1) / splits;
    rps = std::max<int64_t>((rps + 63) / 64 * 64, 64);
    if (narrow) rps = std::min<int64_t>(rps, px::kMaxNarrowSplitRows);
    splits = (int)std::max<int64_t>(1, (n_eff + rps - 1) / rps);
    if ((int64_t)splits * kl > px::kMaxMerge)
        return fail(PX_ERR_BAD_K, "k=" + std::to_string(k) + " over " + std::to_string(n_eff) +
                                      " rows needs more split lists than the merge holds");
    if (splits > max_splits)
        return fail(PX_ERR_ARG, "k=" + std::to_string(k) + " over " + std::to_string(n_eff) +
                                    " rows needs more splits than the scratch holds lists for");
    out->splits = splits;
    out->rps = rps;
    out->groups = groups;
    return PX_OK;
}

// The threshold-collect path (large k, and moderate k on large batches), shared by the
// flat and PQ scans.
//  1. Thresholds from a sample of S rows spread evenly over the corpus: an all-pass collect scan over the sample
//     and a radix select give each query the keys of (about) its r0-th and r1-th smallest
//     sampled rows as a two-rung ladder. r0 is set so that the rows at or below it in the
//     whole corpus are, with high probability, at least k' but not many more: about
//     k' * S / n_eff sampled rows are expected below the true k'-th key, and r0 adds five
//     standard deviations and 5; r1 = 2 r0 + 8 is the fallback.
//  2. One collect scan appends every row at or below its query's threshold.
//  3. The select finishes each query that has every candidate and at least k' of them;
//     the others get a new threshold (next rung, or a tighter one from the candidates) and
//     go round again, alone. Each round either finishes a query or strictly shrinks its
//     candidate set, so the loop ends; nearly every query finishes in the first round.
// Device bytes a collect round's candidate regions may take (retry rounds are split into
// chunks of queries to stay under it; PX_COLLECT_BYTES overrides it, read once), and the
// most queries one collect pass serves (the sample keys take 64 KB and the first round's
// regions up to ~170 KB per query).
int64_t collect_bytes() {
    static const int64_t v = [] {
        const char* e = std::getenv("PX_COLLECT_BYTES");
        return e && *e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)4 << 30;
    }();
    return v;
}
constexpr int64_t kCollectBatch = 16384;
// rows of the threshold sample that seeds a bounded first round (CollectJob::seed_rows)
constexpr int64_t kSeedRows = 512;
// Whether the MFMA collect scan also applies the splits' shared bound (default on;
// PX_COLLECT_SHARED_BOUND=0 turns it off, for measurement; read once).
bool shared_collect_bound() {
    static const bool v = [] {
        const char* e = std::getenv("PX_COLLECT_SHARED_BOUND");
        return !(e && *e == '0');
    }();
    return v;
}

struct CollectJob {
    Workspace* ws = nullptr;
    hipStream_t stream = nullptr;
    Timing* timing = nullptr;
    int* last_rounds = nullptr;
    int64_t nq = 0, kk = 0, n_eff = 0;
    int cus = 1;
    // keys of S rows spread evenly over the n_eff positions (position floor(i n_eff / S))
    // -> ladder rungs r0, r1, thresholds, rung 0
    std::function<int(int64_t S, int r0, int r1)> sample;
    // collect scan over the first *slots query slots (qlist: their query indices, or null
    // for all); with a qlist it may take fewer slots so that the regions stay within
    // max_bytes, and returns how many it took, the regions per slot and their capacity
    std::function<int(int64_t* slots, const int* qlist, double expect, int round,
                      int64_t max_bytes, int64_t* regions, int64_t* cap)>
        scan;
    px::CollectSelectArgs sel{};  // metric, corpus (null: no re-rank), dims, k, outputs
    // The first round's scan bounds itself (the splits' shared bound): no sample, no
    // ladder, every query's threshold +inf; bound_expect sizes its regions.
    bool bound_only = false;
    double bound_expect = 0.0;
    // bound_only with seed_rows > 0: the first round's thresholds come from a sample of
    // seed_rows rows (each query's k'-th smallest sampled key, so at least k' rows of the
    // corpus are at or below it) and the shared bound applies on top. Before the bound
    // tightens, a split's first tiles would otherwise pass about half their rows.
    int64_t seed_rows = 0;
    // set by scan: the shared-bound slots of its launch (null when it applied none) and
    // its regions' smallest dropped keys (null when it keeps none: an overflow retries)
    const int* sel_gbest = nullptr;
    const int* sel_dmin = nullptr;
};

int run_collect(CollectJob& j) {
    Workspace& ws = *j.ws;
    hipStream_t s = j.stream;
    const int64_t nq = j.nq, kk = j.kk, n_eff = j.n_eff;
    PX_TRY(ws.thr_k.reserve(sizeof(int) * nq));
    PX_TRY(ws.thr_p.reserve(sizeof(int) * nq));
    PX_TRY(ws.lad_k.reserve(sizeof(int) * nq * px::kRungs));
    PX_TRY(ws.lad_p.reserve(sizeof(int) * nq * px::kRungs));
    PX_TRY(ws.rung.reserve(sizeof(int) * nq));
    // status[nq]: set by a scan whose stage sync gave up (FlatScanArgs::spin_fail)
    PX_TRY(ws.status.reserve(sizeof(int) * (nq + 1)));
    PX_TRY(j.timing->ensure());
    if (j.timing->enabled) PX_HIP(hipEventRecord(j.timing->ev[0], s));
    PX_HIP(px::launch_fill_int(ws.status.as<int>() + nq, 1, 0, s));

    // expected candidates per query in the first round
    double expect = (double)n_eff;
    if (n_eff > kk && j.bound_only && j.seed_rows > 0) {
        const int64_t S = std::min(n_eff, j.seed_rows);
        const int r0 = (int)std::min<int64_t>(S, kk);
        PX_TRY(j.sample(S, r0, (int)std::min<int64_t>(S, 2 * kk + 8)));
        expect = j.bound_expect;
    } else if (n_eff <= kk || j.bound_only) {
        // every row is a candidate
        PX_HIP(px::launch_fill_int(ws.thr_k.as<int>(), nq, px::kTotalKeyInf, s));
        PX_HIP(px::launch_fill_int(ws.thr_p.as<int>(), nq, 0x7fffffff, s));
        PX_HIP(px::launch_fill_int(ws.rung.as<int>(), nq, px::kRungs, s));
        if (n_eff > kk) expect = j.bound_expect;
    } else {
        const int64_t S = std::max<int64_t>(
            1, std::min<int64_t>({n_eff, (int64_t)16384, 80 * n_eff / kk}));
        const double x = (double)kk * (double)S / (double)n_eff;
        const int r0 = (int)std::min<int64_t>(S, (int64_t)std::ceil(x + 5.0 * std::sqrt(x) + 5.0));
        const int r1 = (int)std::min<int64_t>(S, 2 * (int64_t)r0 + 8);
        // each sampled row stands for n_eff / S rows
        expect = std::min<double>((double)n_eff, (double)(r0 + 4) * (double)n_eff / (double)S);
        PX_TRY(j.sample(S, r0, r1));
    }

    PX_TRY(ws.ensure_status(nq + 1));
    int* h_status = ws.h_status;
    std::vector<int> failing;
    int64_t slots = nq;
    const int* qlist = nullptr;
    for (int round = 0;; ++round) {
        *j.last_rounds = round + 1;
        // the round's slots, in chunks whose candidate regions fit collect_bytes() (only
        // retry rounds, which list their queries, are ever split)
        for (int64_t done = 0; done < slots;) {
            int64_t take = slots - done, regions = 0, cap = 0;
            const int* ql = qlist ? qlist + done : nullptr;
            PX_TRY(j.scan(&take, ql, expect, round, qlist ? collect_bytes() : INT64_MAX, &regions,
                          &cap));
            if (round == 0 && j.timing->enabled) PX_HIP(hipEventRecord(j.timing->ev[1], s));
            int64_t lcap = 1;
            while (lcap < std::max<int64_t>(std::min<int64_t>(regions * cap, px::kMaxCollect),
                                            2 * kk + 1))
                lcap <<= 1;
            lcap = std::min<int64_t>(lcap, px::kMaxCollect);
            // a round bounded by the shared bound holds a few hundred candidates a query and
            // sorts only those below the final bound: 32 KB of LDS lets five selects share a
            // CU where 64 KB let two (more than 4,096 candidates counts as an overflow)
            if (j.sel_gbest) lcap = std::max<int64_t>(std::min<int64_t>(lcap, 4096), 2 * kk + 1);
            // a sampled first round holds about `expect` candidates a query (its threshold
            // sits five standard deviations above the k'-th): where twice that fits 8,192
            // entries the select takes no more (64 KB of LDS: two workgroups a CU, where room
            // for every region full took 128 KB and one; 1M x 128, k = 1000); more is an
            // overflow. Later rounds keep the room of their regions.
            else if (round == 0 && 2.0 * expect + 1 <= 8192.0 && 2 * kk + 1 <= 8192) {
                lcap = std::min<int64_t>(lcap, 8192);
            }

            PX_INTERNAL(lcap >= 1 && lcap <= px::kMaxCollect && (lcap & (lcap - 1)) == 0);
            PX_INTERNAL((size_t)(take * regions) * 4 <= ws.cand_n.cap);
            px::CollectSelectArgs c = j.sel;
            c.dbg = ws.dbg;
            c.cand_keys = ws.cand_k.as<float>();
            c.cand_pos = ws.cand_p.as<int>();
            c.cand_count = ws.cand_n.as<int>();
            c.regions = (int)regions;
            c.cap = (int)cap;
            c.lcap = (int)lcap;
            c.qlist = ql;
            c.thr_key = ws.thr_k.as<int>();
            c.thr_pos = ws.thr_p.as<int>();
            c.ladder_key = ws.lad_k.as<int>();
            c.ladder_pos = ws.lad_p.as<int>();
            c.rung = ws.rung.as<int>();
            c.status = ws.status.as<int>();
            c.kk = (int)kk;
            c.gbest = j.sel_gbest;
            c.gbest_ld = j.nq;
            c.cand_dmin = j.sel_dmin;
            // a scan's stage sync that gave up (status[nq]): the select writes nothing
            c.spin_fail = ws.status.as<int>() + nq;
            PX_HIP(px::launch_collect_select(c, (int)take, s));
            if (round == 0 && j.timing->enabled) PX_HIP(hipEventRecord(j.timing->ev[2], s));
            done += take;
        }
        PX_HIP(px::launch_copy_to_host(ws.status.as<int>(), ws.h_status_dev, nq + 1, s));
        PX_HIP(hipStreamSynchronize(s));
        if (h_status[nq])
            return fail(PX_ERR_DEVICE, "a collect scan's stage sync timed out (no results)");
        // queries of this round still open
        std::vector<int> next;
        if (qlist) {
            for (int q : failing)
                if (h_status[q]) next.push_back(q);
        } else {
            for (int64_t q = 0; q < nq; ++q)
                if (h_status[q]) next.push_back((int)q);
        }
        if (next.empty()) break;
        if (round >= 10000)
            return fail(PX_ERR_ARG, "large-k selection did not converge");  // unreachable
        failing.swap(next);
        PX_TRY(ws.qlist.reserve(sizeof(int) * failing.size()));
        PX_HIP(hipMemcpyAsync(ws.qlist.p, failing.data(), sizeof(int) * failing.size(),
                              hipMemcpyHostToDevice, s));
        qlist = ws.qlist.as<int>();
        slots = (int64_t)failing.size();
        expect = (double)(2 * kk + 1);
    }
    if (j.timing->enabled) {
        if (*j.last_rounds > 1) PX_HIP(hipEventRecord(j.timing->ev[2], s));
        PX_HIP(hipStreamSynchronize(s));
        PX_HIP(hipEventElapsedTime(&j.timing->scan_ms, j.timing->ev[0], j.timing->ev[1]));
        PX_HIP(hipEventElapsedTime(&j.timing->total_ms, j.timing->ev[0], j.timing->ev[2]));
    }
    return PX_OK;
}

// Region capacity of a collect round: 3x the expected candidates spread over the regions,
// at least 2 k' + 1 after the first round (so an overflowing region holds enough to
// tighten from), whole multiples of 32, never more than a region can receive.
// Whether a collect scan of `slots` query slots runs on the vector ALUs.
bool vec_collect(int64_t slots, int64_t dp) {
    int64_t np = 1;  // slots rounded up to the kernel's power of two
    while (np < slots) np <<= 1;
    return slots >= 1 && slots <= px::kVecQueries && dp <= px::kVecMaxDp &&
           np * dp <= px::kVecMaxQueryFloats;
}

int64_t collect_cap(double expect, int64_t regions, int round, int64_t kk, int64_t most) {
    int64_t cap = (int64_t)std::ceil(3.0 * expect / (double)regions);
    if (round > 0) cap = std::max<int64_t>(cap, 2 * kk + 1);
    return std::max<int64_t>(1, std::min<int64_t>((cap + 31) / 32 * 32, most));
}

// Splits and rows per split of an MFMA collect scan of `slots` query slots, qpb of them a
// workgroup (256; the fp16 scan 512).
void collect_splits(int64_t n_eff, int64_t slots, int cus, int64_t* splits, int64_t* rps,
                    int64_t qpb = 256) {
    const int64_t groups = (slots + qpb - 1) / qpb;
    int64_t sp = std::min<int64_t>(choose_flat_splits(n_eff, groups, 1, cus, false),
                                   px::kMaxCollectRegions / 2);
    int64_t r = (n_eff + sp - 1) / sp;
    r = std::max<int64_t>((r + 63) / 64 * 64, 64);
    *splits = std::max<int64_t>(1, (n_eff + r - 1) / r);
    *rps = r;
}

// Whether an MFMA collect scan over `splits` splits applies the shared bound for k'.
bool collect_shared_bound(int64_t splits, int64_t kk) {
    return shared_collect_bound() && std::min<int64_t>(splits, 32) >= kk;
}

// Moderate k' on short corpora stays on the lists, where the sample scan alone adds
// S / n_eff of a scan. With several query chunks (dp > 128) the lists hold up to 16 threshold
// samples' worth of rows (100k x 384 IP, 1,000 queries, k = 16: lists 0.97 ms, sampled
// collect 1.08 ms; k = 32: 0.95 against 0.97). With one chunk the sampled collect scan
// overtakes them far sooner (ms a search, lists against sampled collect, 1,000 queries,
// N(0,1) IP and SIFT-like L2 alike): k = 16: 100k rows 0.44 against 0.44-0.46, 250k 0.84
// against 0.79; k = 32: 20k 0.24 against 0.25, 50k 0.37 against 0.33, 100k 0.52 against
// 0.44; k = 48: 20k 0.30 against 0.25 (4,000 queries: 0.72 against 0.76), 100k 0.61
// against 0.45. The lists' cost grows with k' and the sample's does not: the crossover falls
// near n_eff (k' - 16) = 1.04M rows (k' = 24: 130k rows, 40: 43k, 56: 26k).
bool lists_beat_sample(int64_t n_eff, int64_t kk, int64_t dp) {
    if (kk > 56) return false;
    if (dp > 128) return n_eff < 16 * 16384;
    return kk <= 16 || n_eff * (kk - 16) < 1040000;
}

// Whether a collect batch of nq query slots runs its first round on the shared bound alone
// (no sample, no ladder). Measured on one MI355X against the per-split lists and the
// sampled threshold (ms per batch of device-resident queries):
//   1M x 128 SIFT-like L2, 10,000 queries: k = 10: 22.2 (lists 23.5); k = 16: 22.6 (lists
//     24.7, sampled 24.4); k = 24 (k' = 32): 25.8 and a second round (sampled 24.5)
//   300k x 128, 10,000 queries, k = 10: 7.6 (lists 8.3)
//   1M x 128, 2,000 queries (96 splits), k = 10: 5.1 (lists 5.0): every split's first
//     tile adds up to k' candidates a query
//   100k / 1M x 384 IP, 1,000-4,000 queries, k = 10: 1-2% behind the lists (several query
//     chunks: the keys are tested in the epilogue, not during the next tile's MFMAs)
//   1M x 128 with a 50% / 10% / 2% filter, k = 10: 10.8 / 2.8 / 1.1 on flat_collect_kernel
//     (lists 13.1 / 3.5 / 1.3); on the older scan (flat_scan_kernel's collect mode, rows of
//     other widths) 13.2 / 3.7 against 13.1 / 3.6, so filtered rows take it only at 128
//     padded dims
// so: one 128-dim chunk (filtered: exactly 128), at most 48 splits, k' <= 24 (the bound is
// the k'-th smallest of at most 32 split minima; at k' = 32 it is their largest and prunes
// little).
bool collect_bound_only(int64_t n_eff, int64_t nq, int64_t kk, int64_t dp, int cus,
                        bool filtered) {
    if ((filtered && dp != 128) || dp > 128 || kk > 24 || nq < kCollectMinQueries ||
        vec_collect(nq, dp))
        return false;
    int64_t splits = 1, rps = 64;
    collect_splits(n_eff, std::min(nq, kCollectBatch), cus, &splits, &rps);
    return splits <= 48 && collect_shared_bound(splits, kk);
}

int flat_run_collect_batch(px_flat* f, const float* d_q, int64_t nq, int64_t k, int64_t n_eff,
                           const int* rowidx, int64_t* d_ids, float* d_out, int raw_keys) {
    Workspace& ws = f->ws;
    hipStream_t s = f->stream;
    const int cus = std::max(f->dev.cus, 1);
    // the fp16 scan: rows exact in fp16 (d_xh) and so are this batch's queries (one
    // conversion pass, its verdict read back)
    // (queries checked on the host: no read-back, or no conversion at all)
    const unsigned short* qh = nullptr;
    if (f->scan_f16 && f->d_xh && f->dp == 128 && !vec_collect(nq, f->dp) &&
        ((uintptr_t)d_q & 15) == 0 && f->q_f16 != 0) {
        PX_TRY(ws.qh.reserve(sizeof(unsigned short) * nq * 128));
        PX_TRY(ws.count.reserve(sizeof(int)));
        PX_TRY(ws.ensure_pinned());
        PX_HIP(px::launch_fill_int(ws.count.as<int>(), 1, 0, s));
        PX_HIP(px::launch_to_f16(d_q, nq * 128, ws.qh.as<unsigned short>(), ws.count.as<int>(),
                                 s));
        if (f->q_f16 == 1) {
            qh = ws.qh.as<unsigned short>();
        } else {
            PX_TRY(read_back_int(ws.count.as<int>(), ws.h_count, ws.h_count_dev, s));
            if (*ws.h_count == 0) qh = ws.qh.as<unsigned short>();
        }
    }
    // the vector-ALU scan of a few queries reads the fp16 copy of the rows (half the bytes)
    // and widens it: the same values, whatever the queries hold
    const unsigned short* vh =
        f->scan_f16 && f->d_xh && f->dp == 128 && vec_collect(nq, f->dp) ? f->d_xh : nullptr;
    f->last_f16 = qh != nullptr || vh != nullptr;
    // query slots a workgroup of the (non-dense) MFMA collect scan
    const int64_t qpb = qh                                      ? px::flat_collect16_queries_per_block()
                        : px::collect_resident_queries(f->dp) ? 128
                                                                : 256;
    CollectJob j;
    j.ws = &ws;
    j.stream = s;
    j.timing = &f->timing;
    j.last_rounds = &f->last_rounds;
    f->last_path = vec_collect(nq, f->dp) ? PX_PATH_VECTOR : PX_PATH_COLLECT_SAMPLED;
    j.nq = nq;
    j.kk = k + kReRankMargin;
    j.n_eff = n_eff;
    j.cus = cus;
    j.sample = [&](int64_t S, int r0, int r1) -> int {
        PX_TRY(ws.samp_row.reserve(sizeof(int) * S));
        PX_HIP(px::launch_sample_rows(rowidx, S, n_eff, ws.samp_row.as<int>(), s));
        if (vec_collect(nq, f->dp)) {
            // a few queries: the sampled rows' keys from the vector-ALU scan, row-major
            const int64_t want = std::min<int64_t>(px::kMaxCollectRegions, 4 * (int64_t)cus);
            int64_t rps = (S + want - 1) / want;
            rps = std::max<int64_t>((rps + 63) / 64 * 64, 64);
            PX_TRY(ws.cand_k.reserve(sizeof(float) * nq * S));
            px::FlatScanArgs a{};
            a.dbg = f->ws.dbg;
            a.rows = f->d_rows;
            a.corpus = f->d_x;
            a.norms = f->d_norm;
            a.queries = d_q;
            a.rowidx = ws.samp_row.as<int>();
            a.n_eff = S;
            a.rows_per_split = rps;
            a.dp = (int)f->dp;
            a.nq = (int)nq;
            a.splits = (int)((S + rps - 1) / rps);
            a.metric = f->smetric;
            a.cand_keys = ws.cand_k.as<float>();
            a.dense = 1;
            a.corpus_h = vh;
            PX_HIP(px::launch_flat_vcollect(a, s));
            px::LadderArgs la{};
            la.keys = a.cand_keys;
            la.ld = S;
            la.count = (int)S;
            la.nq = (int)nq;
            la.ranks[0] = r0;
            la.ranks[1] = r1;
            la.ladder_key = ws.lad_k.as<int>();
            la.ladder_pos = ws.lad_p.as<int>();
            la.thr_key = ws.thr_k.as<int>();
            la.thr_pos = ws.thr_p.as<int>();
            la.rung = ws.rung.as<int>();
            PX_HIP(px::launch_ladder(la, s));
            return PX_OK;
        }
        // dense keys of the sample, row-major [query][splits * rps] by position
        const int64_t groups = (nq + 255) / 256;
        int64_t splits = choose_flat_splits(S, groups, 1, cus, false);
        int64_t rps = (S + splits - 1) / splits;
        rps = std::max<int64_t>((rps + 63) / 64 * 64, 64);
        splits = std::max<int64_t>(1, (S + rps - 1) / rps);
        const int64_t ld = splits * rps;
        if (S > px::kMaxLadderEntries)
            return fail(PX_ERR_ARG, "internal: threshold sample too large for the ladder");
        PX_TRY(ws.cand_k.reserve(sizeof(float) * nq * ld));
        px::FlatScanArgs a{};
        a.dbg = f->ws.dbg;
        a.rows = f->d_rows;
        a.corpus = f->d_x;
        a.norms = f->d_norm;
        a.queries = d_q;
        a.rowidx = ws.samp_row.as<int>();
        a.n_eff = S;
        a.rows_per_split = rps;
        a.dp = (int)f->dp;
        a.nq = (int)nq;
        a.splits = (int)splits;
        a.metric = f->smetric;
        a.cand_keys = ws.cand_k.as<float>();
        a.dense = 1;
        a.dense_ld = ld;
        a.spin_fail = ws.status.as<int>() + nq;
        a.spin_limit = f->spin_limit;
        a.corpus_h = qh ? f->d_xh : nullptr;
        a.queries_h = qh;
        a.xcd_major = xcd_major_for(a, 256, std::max(f->dev.cus, 1));
        PX_HIP(px::launch_flat_collect(a, s));
        px::LadderArgs la{};
        la.keys = a.cand_keys;
        la.ld = ld;
        la.count = (int)S;
        la.nq = (int)nq;
        la.ranks[0] = r0;
        la.ranks[1] = r1;
        la.ladder_key = ws.lad_k.as<int>();
        la.ladder_pos = ws.lad_p.as<int>();
        la.thr_key = ws.thr_k.as<int>();
        la.thr_pos = ws.thr_p.as<int>();
        la.rung = ws.rung.as<int>();
        PX_HIP(px::launch_ladder(la, s));
        return PX_OK;
    };
    j.scan = [&](int64_t* take, const int* qlist, double expect, int round, int64_t max_bytes,
                 int64_t* regions, int64_t* cap) -> int {
        int64_t slots = *take, splits = 1, rps = 64;
        if (vec_collect(slots, f->dp)) {
            // a few slots: the vector-ALU scan, one region per (slot, split), up to four
            // workgroups of 512 threads per CU
            const int64_t want = std::min<int64_t>(px::kMaxCollectRegions, 4 * (int64_t)cus);
            rps = (n_eff + want - 1) / want;
            rps = std::max<int64_t>((rps + 63) / 64 * 64, 64);
            splits = std::max<int64_t>(1, (n_eff + rps - 1) / rps);
            *regions = splits;
            *cap = collect_cap(expect, *regions, round, j.kk, rps);
            PX_TRY(ws.cand_k.reserve(sizeof(float) * slots * *regions * *cap));
            PX_TRY(ws.cand_p.reserve(sizeof(int) * slots * *regions * *cap));
            PX_TRY(ws.cand_n.reserve(sizeof(int) * slots * *regions));
            px::FlatScanArgs a{};
            a.dbg = f->ws.dbg;
            a.rows = f->d_rows;
            a.corpus = f->d_x;
            a.norms = f->d_norm;
            a.queries = d_q;
            a.rowidx = rowidx;
            a.n_eff = n_eff;
            a.rows_per_split = rps;
            a.dp = (int)f->dp;
            a.nq = (int)slots;
            a.splits = (int)splits;
            a.metric = f->smetric;
            a.qlist = qlist;
            a.thr_key = ws.thr_k.as<int>();
            a.thr_pos = ws.thr_p.as<int>();
            a.cand_keys = ws.cand_k.as<float>();
            a.cand_pos = ws.cand_p.as<int>();
            a.cand_count = ws.cand_n.as<int>();
            a.cap = (int)*cap;
            a.corpus_h = vh;
            j.sel_dmin = nullptr;
            PX_HIP(px::launch_flat_vcollect(a, s));
            if (round == 0) {
                f->timing.splits = (int)splits;
                f->timing.blocks = (int)splits;
            }
            return PX_OK;
        }
        for (;;) {
            collect_splits(n_eff, slots, cus, &splits, &rps, qpb);
            // two regions per split (one per lane of the pair holding a query), each of
            // which receives at most half the split's rows
            *regions = 2 * splits;
            *cap = collect_cap(expect, *regions, round, j.kk, rps / 2);
            const int64_t per = *regions * (*cap * 8 + 4);
            if (!qlist || slots == 1 || slots * per <= max_bytes) break;
            slots = std::max<int64_t>(1, std::min(slots - 1, max_bytes / per));
        }
        *take = slots;
        PX_TRY(ws.cand_k.reserve(sizeof(float) * slots * *regions * *cap));
        PX_TRY(ws.cand_p.reserve(sizeof(int) * slots * *regions * *cap));
        PX_TRY(ws.cand_n.reserve(sizeof(int) * slots * *regions));
        // rows of one 128-dim chunk (flat_collect_kernel) keep each full region's first cap
        // rows and its smallest dropped key; the older scan rewrites the last slot
        const bool keeps_dmin = f->dp == 128;
        if (keeps_dmin) PX_TRY(ws.cand_d.reserve(sizeof(int) * slots * *regions));
        // every split is non-empty, two regions each, and the launch's regions fit
        PX_INTERNAL(splits * rps >= n_eff && (splits - 1) * rps < n_eff);
        PX_INTERNAL(*regions == 2 * splits && *regions <= px::kMaxCollectRegions);
        PX_INTERNAL(*cap >= 1 && (size_t)(slots * *regions * *cap) * 4 <= ws.cand_k.cap);
        px::FlatScanArgs a{};
        a.dbg = f->ws.dbg;
        a.rows = f->d_rows;
        a.corpus = f->d_x;
        a.norms = f->d_norm;
        a.queries = d_q;
        a.rowidx = rowidx;
        a.n_eff = n_eff;
        a.rows_per_split = rps;
        a.dp = (int)f->dp;
        a.nq = (int)slots;
        a.splits = (int)splits;
        a.metric = f->smetric;
        a.qlist = qlist;
        a.thr_key = ws.thr_k.as<int>();
        a.thr_pos = ws.thr_p.as<int>();
        a.cand_keys = ws.cand_k.as<float>();
        a.cand_pos = ws.cand_p.as<int>();
        a.cand_count = ws.cand_n.as<int>();
        a.cap = (int)*cap;
        a.cand_dmin = keeps_dmin ? ws.cand_d.as<int>() : nullptr;
        j.sel_dmin = a.cand_dmin;
        a.spin_fail = ws.status.as<int>() + j.nq;
        a.spin_limit = f->spin_limit;
        a.corpus_h = qh ? f->d_xh : nullptr;
        a.queries_h = qh;
        // the shared bound needs k' publishing slots (one per split, at most 32); it is
        // applied where the first round has no sampled thresholds (with them it measured
        // no faster on 1M x 128 and 1M x 384, and 11% slower on 100k x 384 at k = 16)
        j.sel_gbest = nullptr;
        if (j.bound_only && collect_shared_bound(splits, j.kk)) {
            PX_TRY(ws.gbest.reserve(sizeof(int) * j.nq * 32));
            PX_HIP(px::launch_fill_int(ws.gbest.as<int>(), j.nq * 32, px::kTotalKeyInf, s));
            a.gbest = ws.gbest.as<int>();
            a.gbest_ld = j.nq;
            a.kl = (int)j.kk;
            j.sel_gbest = a.gbest;
        }
        a.xcd_major = xcd_major_for(a, qpb, std::max(f->dev.cus, 1));
        PX_HIP(px::launch_flat_collect(a, s));
        if (round == 0) {
            f->timing.splits = (int)splits;
            f->timing.blocks = (int)(((slots + qpb - 1) / qpb) * splits);
        }
        return PX_OK;
    };
    if (!vec_collect(nq, f->dp)) {
        // the first round bounds itself: per region (one lane of a split) up to k' rows of
        // the split's first tile and a few after it, twice over (a split that starts ahead
        // of the others of its query tile scans a few tiles before their minima arrive, and
        // a split publishes a tile's minimum while it scans the next), and at least
        // 2 k' + 1 (an overflowing region holds enough to tighten from)
        j.bound_only = collect_bound_only(n_eff, nq, j.kk, f->dp, cus, rowidx != nullptr);
        if (j.bound_only) f->last_path = PX_PATH_COLLECT_BOUNDED;
        // the first round seeded by a 512-row sample: the fp16 scan's row tests in each
        // split's first tiles were a tenth of it (1M x 128, 10,000 queries: 2.73 -> 2.65 ms
        // with the seed's own scan and ladder); the fp32 scan hides them behind its MFMAs but
        // its select sorts fewer candidates (19.09 -> 19.01 ms a batch)
        if (j.bound_only) j.seed_rows = kSeedRows;
        int64_t splits = 1, rps = 64;
        collect_splits(n_eff, nq, cus, &splits, &rps, qpb);
        j.bound_expect = (double)(2 * splits) *
                         (double)std::max<int64_t>(2 * (j.kk + 48), 2 * j.kk + 1) / 3.0;
    }
    j.sel.rowidx = rowidx;
    j.sel.k = (int)k;
    j.sel.metric = f->smetric;
    j.sel.corpus = f->d_x;
    j.sel.queries = d_q;
    j.sel.dim = (int)f->dim;
    j.sel.dp = (int)f->dp;
    j.sel.out_ids = d_ids;
    j.sel.out_dists = d_out;
    j.sel.raw_keys = raw_keys;
    return run_collect(j);
}

// k past PX_MAX_K (px_sort.hip): every key of a chunk of queries in the reference's
// arithmetic, one stable radix sort by (query, key), the first k of each query finished and
// padded. Chunks of queries whose keys and sort buffers fit collect_bytes().
int run_full_sort(Workspace& ws, hipStream_t s, Timing& timing, int64_t nq, int64_t k,
                  int64_t n_eff, const int* rowidx, int metric, int raw_keys,
                  const std::function<int(int64_t q0, int qc, float* keys)>& keys_of,
                  int64_t* d_ids, float* d_out) {
    PX_TRY(timing.ensure());
    if (timing.enabled) PX_HIP(hipEventRecord(timing.ev[0], s));
    const int64_t rows = std::max<int64_t>(n_eff, 1);
    const int64_t per_query = rows * (4 + 2 * 8 + 2 * 4) + 4096;
    const int64_t qc = std::max<int64_t>(
        1, std::min<int64_t>({nq, collect_bytes() / per_query, 65535, INT32_MAX / rows}));
    PX_TRY(ws.cand_k.reserve(sizeof(float) * (size_t)(qc * rows)));
    const size_t sb = px::full_sort_scratch_bytes(n_eff, (int)qc);
    PX_TRY(ws.sort_scratch.reserve(sb));
    for (int64_t q0 = 0; q0 < nq; q0 += qc) {
        const int c = (int)std::min(qc, nq - q0);
        if (n_eff > 0) PX_TRY(keys_of(q0, c, ws.cand_k.as<float>()));
        PX_HIP(px::launch_full_sort(ws.cand_k.as<float>(), n_eff, c, rowidx, k, metric, raw_keys,
                                    ws.sort_scratch.p, ws.sort_scratch.cap, d_ids + q0 * k,
                                    d_out + q0 * k, s));
    }
    if (timing.enabled) {
        PX_HIP(hipEventRecord(timing.ev[1], s));
        PX_HIP(hipEventRecord(timing.ev[2], s));
    }
    PX_HIP(hipStreamSynchronize(s));
    if (timing.enabled) {
        PX_HIP(hipEventElapsedTime(&timing.scan_ms, timing.ev[0], timing.ev[1]));
        PX_HIP(hipEventElapsedTime(&timing.total_ms, timing.ev[0], timing.ev[2]));
    }
    return PX_OK;
}

// Batches of at most kCollectBatch queries, one after another.
int flat_run_collect(px_flat* f, const float* d_q, int64_t nq, int64_t k, int64_t n_eff,
                     const int* rowidx, int64_t* d_ids, float* d_out, int raw_keys) {
    int rounds = 0;
    bool all_f16 = true;
    for (int64_t b0 = 0; b0 < nq; b0 += kCollectBatch) {
        const int64_t b = std::min(kCollectBatch, nq - b0);
        PX_TRY(flat_run_collect_batch(f, d_q + b0 * f->dp, b, k, n_eff, rowidx, d_ids + b0 * k,
                                      d_out + b0 * k, raw_keys));
        rounds = std::max(rounds, f->last_rounds);
        all_f16 = all_f16 && f->last_f16;
    }
    f->last_rounds = rounds;
    f->last_f16 = all_f16 && nq > 0;
    return PX_OK;
}

// Device buffers of a list scan: split lists [nq][splits][kl] (key, position), the shared
// bounds gtau [nq] and gbest [32][nq] and the scan's stage-sync give-up word spin (all
// cleared by the list prologue); verdict_h / verdict_dev: two mapped host ints where the
// merge stores the search's finiteness and give-up verdicts, or null (no pinned memory: the
// give-up word is read back by a copy).
struct ListBufs {
    float* part_k;
    int* part_i;
    int* gtau;
    int* gbest;
    int* spin;
    int* verdict_h;
    int* verdict_dev;
};

// The per-split list path: fused MFMA scan with per-split lists, then the merge (re-rank in
// the reference's arithmetic, finish, pad). Waits for the stream. timed: record the
// handle's HIP events (created beforehand).
// qh: the queries in fp16 when they and the rows are exact in fp16 (the fp16 scan), or null.
int flat_run_lists(px_flat* f, const float* d_q, int64_t nq, int64_t k, int64_t n_eff,
                   const int* rowidx, const ListPlan& lp, int kl, const ListBufs& b,
                   int64_t* d_ids, float* d_out, int raw_keys, bool timed,
                   const PendingCheck* chk = nullptr, const unsigned short* qh = nullptr) {
    hipStream_t s = f->stream;
    const int splits = lp.splits;
    const int64_t rps = lp.rps, groups = lp.groups;
    int seq = 0;
    int* d_flag = nullptr;
    if (chk) {
        PX_TRY(next_finite_seq(f->ws, s, &seq));
        d_flag = f->ws.fflag.as<int>();
    }
    PX_HIP(px::launch_list_prologue(chk ? chk->x : nullptr, chk ? chk->count : 0, d_flag, seq,
                                    b.gtau, nq, b.gbest, nq * 32, b.spin, s));
    if (timed) PX_HIP(hipEventRecord(f->timing.ev[0], s));

    px::FlatScanArgs a{};
    a.dbg = f->ws.dbg;
    a.rows = f->d_rows;
    a.corpus = f->d_x;
    a.norms = f->d_norm;
    a.queries = d_q;
    a.rowidx = rowidx;
    a.n_eff = n_eff;
    a.rows_per_split = rps;
    a.dp = (int)f->dp;
    a.nq = (int)nq;
    a.kl = kl;
    a.splits = splits;
    a.metric = f->smetric;
    a.part_keys = b.part_k;
    a.part_ids = b.part_i;
    a.gtau = b.gtau;
    a.gbest = b.gbest;
    a.gbest_ld = nq;
    a.abort = d_flag;
    a.abort_seq = seq;
    a.spin_fail = b.spin;
    a.spin_limit = f->spin_limit;
    a.xcd_major = xcd_major_for(
        a, px::flat_list_queries_per_block(px::flat_list_capacity(kl), f->dp), std::max(f->dev.cus, 1));
    a.corpus_h = qh ? f->d_xh : nullptr;
    a.queries_h = qh;
    if (n_eff > 0) PX_HIP(px::launch_flat_scan(a, s));
    if (timed) PX_HIP(hipEventRecord(f->timing.ev[1], s));

    PX_INTERNAL(n_eff == 0 || ((int64_t)splits * rps >= n_eff && (int64_t)splits * kl <= px::kMaxMerge));
    px::MergeArgs mg{};
    mg.dbg = f->ws.dbg;
    mg.part_keys = a.part_keys;
    mg.part_ids = a.part_ids;
    mg.rowidx = rowidx;
    mg.width = n_eff > 0 ? splits * kl : 0;
    mg.bound = b.gtau;
    mg.gbest = b.gbest;
    mg.gbest_ld = nq;
    mg.splits = splits;
    mg.nq = (int)nq;
    mg.kl = kl;
    mg.k = (int)k;
    mg.metric = f->smetric;
    mg.corpus = f->d_x;
    mg.queries = d_q;
    mg.dim = (int)f->dim;
    mg.dp = (int)f->dp;
    mg.out_ids = d_ids;
    mg.out_dists = d_out;
    mg.raw_keys = raw_keys;
    mg.abort = d_flag;
    mg.abort_seq = seq;
    mg.spin_fail = b.spin;
    mg.verdict = b.verdict_dev;
    PX_HIP(px::launch_merge(mg, s));
    if (timed) PX_HIP(hipEventRecord(f->timing.ev[2], s));
    PX_HIP(hipStreamSynchronize(s));
    // a failed check made the scan and merge no-ops; a stage wait that gave up, the merge
    int gave_up = 0;
    if (b.verdict_h) {
        if (d_flag && b.verdict_h[0] == seq) return nonfinite_error();
        gave_up = b.verdict_h[1];
    } else {
        if (d_flag) return fail(PX_ERR_ARG, "internal: a pending check needs the verdicts");
        PX_TRY(read_back_int(b.spin, &gave_up, nullptr, s));
    }
    if (gave_up)
        return fail(PX_ERR_DEVICE, "a list scan's stage sync timed out (no results)");
    if (timed) {
        PX_HIP(hipEventElapsedTime(&f->timing.scan_ms, f->timing.ev[0], f->timing.ev[1]));
        PX_HIP(hipEventElapsedTime(&f->timing.total_ms, f->timing.ev[0], f->timing.ev[2]));
        f->timing.splits = splits;
        f->timing.blocks = (int)(groups * splits);
    }
    return PX_OK;
}

// Runs the device pipeline. d_q: [nq][dp] on device. Outputs on device.
int flat_run_paths(px_flat* f, const float* d_q, int64_t nq, int64_t k, const uint8_t* d_mask,
                   int64_t* d_ids, float* d_out, int raw_keys, const PendingCheck* chk);

// chk: device queries whose finiteness check has not run yet (PendingCheck), or null.
int flat_run(px_flat* f, const float* d_q, int64_t nq, int64_t k, const uint8_t* d_mask,
             int64_t* d_ids, float* d_out, int raw_keys, const PendingCheck* chk = nullptr) {
    PX_TRY(debug_begin(f->ws, f->stream));
    return debug_end(f->ws, f->stream,
                     flat_run_paths(f, d_q, nq, k, d_mask, d_ids, d_out, raw_keys, chk));
}

int flat_run_paths(px_flat* f, const float* d_q, int64_t nq, int64_t k, const uint8_t* d_mask,
                   int64_t* d_ids, float* d_out, int raw_keys, const PendingCheck* chk) {
    Workspace& ws = f->ws;
    hipStream_t s = f->stream;
    int64_t n_eff = f->d_rows;
    const int* rowidx = nullptr;
    auto check_now = [&]() -> int {
        if (!chk) return PX_OK;
        const PendingCheck c = *chk;
        chk = nullptr;
        return check_device_finite(ws, c.x, c.count, s);
    };
    if (d_mask) {
        PX_TRY(check_now());
        PX_TRY(compact_mask(ws, d_mask, f->d_rows, s, &n_eff, &rowidx));
    }
    f->last_rounds = 0;
    f->last_path = PX_PATH_LISTS;
    f->last_f16 = false;
    if (k > PX_MAX_K) {
        PX_TRY(check_now());
        f->last_path = PX_PATH_FULL_SORT;
        return run_full_sort(ws, s, f->timing, nq, k, n_eff, rowidx, f->smetric, raw_keys,
                             [&](int64_t q0, int qc, float* keys) -> int {
                                 PX_HIP(px::launch_flat_exact_keys(
                                     f->d_x, d_q + q0 * f->dp, rowidx, n_eff, qc, (int)f->dim,
                                     (int)f->dp, f->smetric, keys, s));
                                 return PX_OK;
                             },
                             d_ids, d_out);
    }
    // lists for batches of moderate size and small k; the collect path for large k, for
    // larger k on large batches, and for the few-query batches the vector-ALU scan serves
    const int64_t kk = k + kReRankMargin;
    const bool collect =
        kk > px::kMaxList ||
        (k >= collect_from_k() && nq >= kCollectMinQueries && !lists_beat_sample(n_eff, kk, f->dp)) ||
        vec_collect(nq, f->dp) ||
        collect_bound_only(n_eff, nq, kk, f->dp, std::max(f->dev.cus, 1), rowidx != nullptr);
    if (collect && n_eff > 0) {
        PX_TRY(check_now());
        return flat_run_collect(f, d_q, nq, k, n_eff, rowidx, d_ids, d_out, raw_keys);
    }

    const int kl = (int)std::min<int64_t>(px::kMaxList, k + kReRankMargin);
    // the fp16 scan where the rows are exact in fp16 and so are the queries: one pass
    // converts them and flags any value that is not exact (and, with a finiteness check
    // still pending, any that is not finite), its verdict read back before the scan. On
    // fewer rows the read-back would cost about what the fp16 scan saves.
    const unsigned short* qh = nullptr;
    if (f->scan_f16 && f->d_xh && f->dp == 128 && n_eff >= kF16ListMinRows &&
        ((uintptr_t)d_q & 15) == 0 && f->q_f16 != 0) {
        PX_TRY(ws.qh.reserve(sizeof(unsigned short) * nq * 128));
        PX_TRY(ws.count.reserve(sizeof(int)));
        PX_TRY(ws.ensure_pinned());
        int* flag = ws.count.as<int>();
        const bool pending = chk != nullptr;
        if (chk) {
            PX_HIP(px::launch_nonfinite_check(chk->x, chk->count, flag, s));  // bit 0
            chk = nullptr;
        } else {
            PX_HIP(px::launch_fill_int(flag, 1, 0, s));
        }
        PX_HIP(px::launch_to_f16(d_q, nq * 128, ws.qh.as<unsigned short>(), flag, s, 2));
        if (f->q_f16 == 1 && !pending) {
            qh = ws.qh.as<unsigned short>();  // checked on the host: no read-back
        } else {
            PX_TRY(read_back_int(flag, ws.h_count, ws.h_count_dev, s));
            if (*ws.h_count & 1) return nonfinite_error();
            if (!(*ws.h_count & 2)) qh = ws.qh.as<unsigned short>();
        }
    }
    f->last_f16 = qh != nullptr;
    ListPlan lp;
    PX_TRY(plan_list_scan(n_eff, nq, kl, f->dp, f->dev.cus, &lp, k));
    PX_TRY(ws.part_k.reserve(sizeof(float) * nq * lp.splits * kl));
    PX_TRY(ws.part_i.reserve(sizeof(int) * nq * lp.splits * kl));
    PX_TRY(ws.gtau.reserve(sizeof(int) * nq));
    PX_TRY(ws.gbest.reserve(sizeof(int) * nq * 32));
    PX_TRY(ws.spinw.reserve(sizeof(int)));
    PX_TRY(ws.ensure_pinned());
    PX_TRY(f->timing.ensure());
    ListBufs b{ws.part_k.as<float>(), ws.part_i.as<int>(), ws.gtau.as<int>(),
               ws.gbest.as<int>(),    ws.spinw.as<int>(),  ws.h_count,
               ws.h_count_dev};
    return flat_run_lists(f, d_q, nq, k, n_eff, rowidx, lp, kl, b, d_ids, d_out, raw_keys,
                          f->timing.enabled, chk, qh);
}

void host_padding(int metric, int64_t nq, int64_t k, int64_t* ids, float* out, int raw_keys) {
    for (int64_t i = 0; i < nq * k; ++i) {
        ids[i] = -1;
        out[i] = raw_keys ? FLT_MAX : (metric == 0 ? FLT_MAX : -FLT_MAX);
    }
}

int check_search_args(const void* idx, const void* queries, int64_t nq, int64_t k,
                      const void* ids, const void* dists) {
    if (!idx) return fail(PX_ERR_ARG, "null index handle");
    if (nq < 0) return fail(PX_ERR_ARG, "nq must be >= 0");
    if (k < 0) return fail(PX_ERR_BAD_K, "k must be >= 0");
    if (k > 0 && nq > 0 && (!queries || !ids || !dists))
        return fail(PX_ERR_ARG, "null query or output pointer");
    return PX_OK;
}

// Host-pointer search: upload, run, download.
int flat_search_host(px_flat* f, int metric, const float* queries, int64_t nq, int64_t k,
                     const uint8_t* mask, int64_t* out_ids, float* out_d, int raw_keys) {
    // small batches test fp16 exactness in the finiteness pass (a few microseconds), sparing
    // the fp16 scans' device read-back; on large ones that pass would cost more than it
    bool f16_exact = false;
    const bool small = nq * f->dim <= 65536;
    if (!(small ? finite_and_f16(queries, nq * f->dim, &f16_exact)
                : all_finite(queries, nq * f->dim)))
        return fail(PX_ERR_NONFINITE, "query must not contain NaN or infinite values");
    std::lock_guard<std::mutex> lock(f->mu);
    f->smetric = metric;
    // the fp16 scans need no read-back of their device check for these queries
    struct HintReset {
        px_flat* f;
        ~HintReset() { f->q_f16 = -1; }
    } hint_reset{f};
    f->q_f16 = small ? (f16_exact ? 1 : 0) : -1;
    if (f->n == 0) {
        host_padding(metric, nq, k, out_ids, out_d, raw_keys);
        return PX_OK;
    }
    PX_TRY(flat_sync(f));
    Workspace& ws = f->ws;
    hipStream_t s = f->stream;
    const float* d_q = nullptr;
    PX_TRY(upload_queries(ws, queries, nq, f->dim, f->dp, s, &d_q));
    const uint8_t* d_mask = nullptr;
    if (mask) {
        PX_TRY(ws.mask.reserve(f->d_rows));
        PX_HIP(hipMemcpyAsync(ws.mask.p, mask, f->d_rows, hipMemcpyHostToDevice, s));
        d_mask = ws.mask.as<uint8_t>();
    }
    PX_TRY(ws.out_ids.reserve(sizeof(int64_t) * nq * k));
    PX_TRY(ws.out_d.reserve(sizeof(float) * nq * k));
    PX_TRY(flat_run(f, d_q, nq, k, d_mask, ws.out_ids.as<int64_t>(), ws.out_d.as<float>(),
                    raw_keys));
    return download_results(ws, nq, k, s, out_ids, out_d);
}

// ---- PQ ----------------------------------------------------------------------------
int pq_bind(px_pq* p) {
    PX_TRY(bind_device(p->dev));
    if (!p->stream) PX_HIP(hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking));
    return PX_OK;
}

int pq_sync(px_pq* p) {
    PX_TRY(pq_bind(p));
    if (!p->books_on_device) {
        if (!p->d_books) PX_HIP(dev_malloc(&p->d_books, sizeof(float) * p->codebooks.size()));
        PX_HIP(hipMemcpyAsync(p->d_books, p->codebooks.data(), sizeof(float) * p->codebooks.size(),
                              hipMemcpyHostToDevice, p->stream));
        PX_HIP(hipStreamSynchronize(p->stream));
        p->books_on_device = true;
    }
    const int64_t add = p->n - p->d_rows;
    if (add <= 0) return PX_OK;
    if (p->n > p->d_cap) {
        const int64_t cap = std::max<int64_t>({p->n, p->d_cap * 2, 4096});
        uint8_t* nc = nullptr;
        PX_HIP(dev_malloc(&nc, (size_t)(cap * p->m)));
        if (p->d_rows)
            PX_HIP(hipMemcpyAsync(nc, p->d_codes, (size_t)(p->d_rows * p->m),
                                  hipMemcpyDeviceToDevice, p->stream));
        PX_HIP(hipStreamSynchronize(p->stream));
        dev_free(p->d_codes);
        p->d_codes = nc;
        p->d_cap = cap;
    }
    PX_HIP(hipMemcpyAsync(p->d_codes + p->d_rows * p->m, p->codes.data() + p->d_rows * p->m,
                          (size_t)(add * p->m), hipMemcpyHostToDevice, p->stream));
    PX_HIP(hipStreamSynchronize(p->stream));
    p->d_rows = p->n;
    return PX_OK;
}

// Device buffer owned by one call.
struct TmpBuf {
    void* p = nullptr;
    ~TmpBuf() { dev_free(p); }
    int alloc(size_t bytes) {
        PX_HIP(dev_malloc(&p, std::max<size_t>(bytes, 16)));
        return PX_OK;
    }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};

// PQ training on the GPU (pq.rs:54-193): the host plans (sample, initial centroids,
// generator states) and gathers the sample sub-major; the Lloyd iterations run on the
// device. Bit-identical to pq_train_host. Caller holds p->mu.
int pq_train_device(px_pq* p, const float* training, int64_t n_all, int64_t iters,
                    int64_t train_sample, uint64_t seed, float* books) {
    const int64_t m = p->m, d = p->dsub;
    px::PqTrainPlan plan;
    px::pq_train_plan(n_all, m, p->nbits, train_sample, seed, &plan);
    const int64_t n = plan.n, ks = plan.ks;
    std::vector<float> sub((size_t)(m * n * d));
    px::pq_gather_sample(training, p->dim, m, plan, sub.data());
    for (int64_t s = 0; s < m; ++s)
        for (int64_t c = 0; c < ks; ++c)
            std::memcpy(books + (s * ks + c) * d, sub.data() + (s * n + plan.init_rows[s * ks + c]) * d,
                        sizeof(float) * d);
    if (iters == 0) return PX_OK;
    PX_TRY(pq_bind(p));
    hipStream_t st = p->stream;
    TmpBuf data, cents, asg, counts, rng;
    PX_TRY(data.alloc(sizeof(float) * sub.size()));
    PX_TRY(cents.alloc(sizeof(float) * m * ks * d));
    PX_TRY(asg.alloc((size_t)(m * px::pq_train_asg_pitch(n))));
    PX_TRY(counts.alloc(sizeof(int) * m * ks));
    PX_TRY(rng.alloc(sizeof(uint64_t) * m));
    PX_HIP(hipMemcpyAsync(data.p, sub.data(), sizeof(float) * sub.size(), hipMemcpyHostToDevice, st));
    PX_HIP(hipMemcpyAsync(cents.p, books, sizeof(float) * m * ks * d, hipMemcpyHostToDevice, st));
    PX_HIP(hipMemcpyAsync(rng.p, plan.rng_after_init.data(), sizeof(uint64_t) * m,
                          hipMemcpyHostToDevice, st));
    for (int64_t it = 0; it < iters; ++it)
        PX_HIP(px::launch_pq_train_iteration(data.as<float>(), n, (int)d, (int)ks, (int)m,
                                             cents.as<float>(), asg.as<uint8_t>(), counts.as<int>(),
                                             rng.as<uint64_t>(), st));
    PX_HIP(hipMemcpyAsync(books, cents.p, sizeof(float) * m * ks * d, hipMemcpyDeviceToHost, st));
    PX_HIP(hipStreamSynchronize(st));
    return PX_OK;
}

// PQ encoding on the GPU (pq.rs:107-121, 266-284), in chunks of 2^20 rows. Caller holds
// p->mu.
int pq_encode_device(px_pq* p, const float* vectors, int64_t n, uint8_t* codes) {
    PX_TRY(pq_bind(p));
    hipStream_t st = p->stream;
    const int64_t chunk = std::min<int64_t>(n, (int64_t)1 << 20);
    TmpBuf books, vec, out;
    PX_TRY(books.alloc(sizeof(float) * p->codebooks.size()));
    PX_TRY(vec.alloc(sizeof(float) * chunk * p->dim));
    PX_TRY(out.alloc((size_t)(chunk * p->m)));
    PX_HIP(hipMemcpyAsync(books.p, p->codebooks.data(), sizeof(float) * p->codebooks.size(),
                          hipMemcpyHostToDevice, st));
    for (int64_t r0 = 0; r0 < n; r0 += chunk) {
        const int64_t rows = std::min(chunk, n - r0);
        PX_HIP(hipMemcpyAsync(vec.p, vectors + r0 * p->dim, sizeof(float) * rows * p->dim,
                              hipMemcpyHostToDevice, st));
        PX_HIP(px::launch_pq_encode(vec.as<float>(), rows, (int)p->dim, (int)p->dsub, (int)p->ks,
                                    (int)p->m, books.as<float>(), out.as<uint8_t>(), st));
        PX_HIP(hipMemcpyAsync(codes + r0 * p->m, out.p, (size_t)(rows * p->m),
                              hipMemcpyDeviceToHost, st));
        PX_HIP(hipStreamSynchronize(st));
    }
    return PX_OK;
}

// k past the lists: the threshold-collect path with exact ADC keys (no re-rank, k' = k).
int pq_run_collect_batch(px_pq* p, const float* d_q, int64_t nq, int64_t k, int64_t n_eff,
                         const int* rowidx, int64_t* d_ids, float* d_out) {
    Workspace& ws = p->ws;
    hipStream_t s = p->stream;
    const int cus = std::max(p->dev.cus, 1);
    const int waves = px::pq_lists_per_split();
    // splits of whole blocks of rows (each wave of a workgroup takes 64 of every rg rows, so
    // that a region of cap rps / waves can take all of its wave's rows)
    const int64_t rg = px::pq_rows_per_block_step();
    const int64_t qpb = px::pq_queries_per_block((int)p->m, (int)p->ks);
    auto base_args = [&]() {
        px::PqScanArgs a{};
        a.dbg = p->ws.dbg;
        a.rows = p->d_rows;
        a.codes = p->d_codes;
        a.codebooks = p->d_books;
        a.queries = d_q;
        a.dim = (int)p->dim;
        a.m = (int)p->m;
        a.ks = (int)p->ks;
        a.dsub = (int)p->dsub;
        a.metric = p->metric;
        return a;
    };
    auto plan = [&](int64_t rows, int64_t slots, int64_t* splits, int64_t* rps) {
        const int64_t groups = (slots + qpb - 1) / qpb;
        *splits = std::min<int64_t>(choose_splits(rows, groups, waves, 1, cus, 4096),
                                    px::kMaxCollectRegions / waves);
        *rps = (rows + *splits - 1) / *splits;
        *rps = std::max<int64_t>((*rps + rg - 1) / rg * rg, rg);
        *splits = std::max<int64_t>(1, (rows + *rps - 1) / *rps);
    };
    CollectJob j;
    j.ws = &ws;
    j.stream = s;
    j.timing = &p->timing;
    j.last_rounds = &p->last_rounds;
    j.nq = nq;
    j.kk = k;
    j.n_eff = n_eff;
    j.cus = cus;
    j.sample = [&](int64_t S, int r0, int r1) -> int {
        PX_TRY(ws.samp_row.reserve(sizeof(int) * S));
        PX_HIP(px::launch_sample_rows(rowidx, S, n_eff, ws.samp_row.as<int>(), s));
        PX_TRY(ws.cand_k.reserve(sizeof(float) * nq * S));
        int64_t splits, rps;
        plan(S, nq, &splits, &rps);
        px::PqScanArgs a = base_args();
        a.rowidx = ws.samp_row.as<int>();
        a.n_eff = S;
        a.rows_per_split = rps;
        a.nq = (int)nq;
        a.splits = (int)splits;
        a.cand_keys = ws.cand_k.as<float>();
        a.dense = 1;
        PX_HIP(px::launch_pq_collect(a, s));
        px::LadderArgs la{};
        la.keys = a.cand_keys;
        la.ld = S;
        la.count = (int)S;
        la.nq = (int)nq;
        la.ranks[0] = r0;
        la.ranks[1] = r1;
        la.ladder_key = ws.lad_k.as<int>();
        la.ladder_pos = ws.lad_p.as<int>();
        la.thr_key = ws.thr_k.as<int>();
        la.thr_pos = ws.thr_p.as<int>();
        la.rung = ws.rung.as<int>();
        PX_HIP(px::launch_ladder(la, s));
        return PX_OK;
    };
    j.scan = [&](int64_t* take, const int* qlist, double expect, int round, int64_t max_bytes,
                 int64_t* regions, int64_t* cap) -> int {
        int64_t slots = *take, splits = 1, rps = 256;
        for (;;) {
            plan(n_eff, slots, &splits, &rps);
            // one region per wave of a split; a wave takes 64 of every rg rows
            *regions = splits * waves;
            *cap = collect_cap(expect, *regions, round, j.kk, rps / waves);
            const int64_t per = *regions * *cap * 8;
            if (!qlist || slots == 1 || slots * per <= max_bytes) break;
            slots = std::max<int64_t>(1, std::min(slots - 1, max_bytes / per));
        }
        *take = slots;
        PX_TRY(ws.cand_k.reserve(sizeof(float) * slots * *regions * *cap));
        PX_TRY(ws.cand_p.reserve(sizeof(int) * slots * *regions * *cap));
        PX_TRY(ws.cand_n.reserve(sizeof(int) * slots * *regions));
        px::PqScanArgs a = base_args();
        a.rowidx = rowidx;
        a.n_eff = n_eff;
        a.rows_per_split = rps;
        a.nq = (int)slots;
        a.splits = (int)splits;
        a.qlist = qlist;
        a.thr_key = ws.thr_k.as<int>();
        a.thr_pos = ws.thr_p.as<int>();
        a.cand_keys = ws.cand_k.as<float>();
        a.cand_pos = ws.cand_p.as<int>();
        a.cand_count = ws.cand_n.as<int>();
        a.cap = (int)*cap;
        PX_HIP(px::launch_pq_collect(a, s));
        if (round == 0) {
            p->timing.splits = (int)splits;
            p->timing.blocks = (int)(((slots + qpb - 1) / qpb) * splits);
        }
        return PX_OK;
    };
    j.sel.rowidx = rowidx;
    j.sel.k = (int)k;
    j.sel.metric = p->metric;
    j.sel.corpus = nullptr;  // ADC keys are the reference's already
    j.sel.out_ids = d_ids;
    j.sel.out_dists = d_out;
    j.sel.raw_keys = 0;
    return run_collect(j);
}

int pq_run_collect(px_pq* p, const float* d_q, int64_t nq, int64_t k, int64_t n_eff,
                   const int* rowidx, int64_t* d_ids, float* d_out) {
    int rounds = 0;
    for (int64_t b0 = 0; b0 < nq; b0 += kCollectBatch) {
        const int64_t b = std::min(kCollectBatch, nq - b0);
        PX_TRY(pq_run_collect_batch(p, d_q + b0 * p->dim, b, k, n_eff, rowidx, d_ids + b0 * k,
                                    d_out + b0 * k));
        rounds = std::max(rounds, p->last_rounds);
    }
    p->last_rounds = rounds;
    return PX_OK;
}

int pq_run_paths(px_pq* p, const float* d_q, int64_t nq, int64_t k, const uint8_t* d_mask,
                 int64_t* d_ids, float* d_out);

int pq_run(px_pq* p, const float* d_q, int64_t nq, int64_t k, const uint8_t* d_mask,
           int64_t* d_ids, float* d_out) {
    PX_TRY(debug_begin(p->ws, p->stream));
    return debug_end(p->ws, p->stream, pq_run_paths(p, d_q, nq, k, d_mask, d_ids, d_out));
}

int pq_run_paths(px_pq* p, const float* d_q, int64_t nq, int64_t k, const uint8_t* d_mask,
                 int64_t* d_ids, float* d_out) {
    Workspace& ws = p->ws;
    hipStream_t s = p->stream;
    int64_t n_eff = p->d_rows;
    const int* rowidx = nullptr;
    if (d_mask) PX_TRY(compact_mask(ws, d_mask, p->d_rows, s, &n_eff, &rowidx));

    p->last_rounds = 0;
    if (k > PX_MAX_K) {
        const int waves = px::pq_lists_per_split();
        const int64_t rg = px::pq_rows_per_block_step();
        const int64_t qpb = px::pq_queries_per_block((int)p->m, (int)p->ks);
        const int cus = std::max(p->dev.cus, 1);
        return run_full_sort(
            ws, s, p->timing, nq, k, n_eff, rowidx, p->metric, 0,
            [&](int64_t q0, int qc, float* keys) -> int {
                // the ADC scan's dense mode: every key, in the reference's order
                const int64_t groups = (qc + qpb - 1) / qpb;
                int64_t splits = std::min<int64_t>(
                    choose_splits(n_eff, groups, waves, 1, cus, 4096), px::kMaxCollectRegions / waves);
                int64_t rps = (n_eff + splits - 1) / splits;
                rps = std::max<int64_t>((rps + rg - 1) / rg * rg, rg);
                splits = std::max<int64_t>(1, (n_eff + rps - 1) / rps);
                px::PqScanArgs a{};
                a.dbg = p->ws.dbg;
                a.rows = p->d_rows;
                a.codes = p->d_codes;
                a.codebooks = p->d_books;
                a.queries = d_q + q0 * p->dim;
                a.dim = (int)p->dim;
                a.m = (int)p->m;
                a.ks = (int)p->ks;
                a.dsub = (int)p->dsub;
                a.metric = p->metric;
                a.rowidx = rowidx;
                a.n_eff = n_eff;
                a.rows_per_split = rps;
                a.nq = qc;
                a.splits = (int)splits;
                a.cand_keys = keys;
                a.dense = 1;
                PX_HIP(px::launch_pq_collect(a, s));
                return PX_OK;
            },
            d_ids, d_out);
    }
    if (k > px::kMaxList && n_eff > 0) return pq_run_collect(p, d_q, nq, k, n_eff, rowidx, d_ids, d_out);
    const int kl = (int)std::min<int64_t>(k, px::kMaxList);
    const int lists = px::pq_lists_per_split();
    const int64_t rg = px::pq_rows_per_block_step();
    const int64_t qpb = px::pq_queries_per_block((int)p->m, (int)p->ks);
    const int64_t groups = (nq + qpb - 1) / qpb;
    int splits = choose_splits(n_eff, groups, lists, kl, p->dev.cus, 4096);
    int64_t rps = (n_eff + splits - 1) / splits;
    rps = std::max<int64_t>((rps + rg - 1) / rg * rg, rg);
    splits = (int)std::max<int64_t>(1, (n_eff + rps - 1) / rps);
    const int64_t width = (int64_t)splits * lists * kl;

    PX_TRY(ws.part_k.reserve(sizeof(float) * nq * width));
    PX_TRY(ws.part_i.reserve(sizeof(int) * nq * width));
    PX_TRY(p->timing.ensure());
    if (p->timing.enabled) PX_HIP(hipEventRecord(p->timing.ev[0], s));
    px::PqScanArgs a{};
    a.dbg = p->ws.dbg;
    a.rows = p->d_rows;
    a.codes = p->d_codes;
    a.codebooks = p->d_books;
    a.queries = d_q;
    a.rowidx = rowidx;
    a.n_eff = n_eff;
    a.rows_per_split = rps;
    a.dim = (int)p->dim;
    a.m = (int)p->m;
    a.ks = (int)p->ks;
    a.dsub = (int)p->dsub;
    a.nq = (int)nq;
    a.kl = kl;
    a.splits = splits;
    a.metric = p->metric;
    a.part_keys = ws.part_k.as<float>();
    a.part_ids = ws.part_i.as<int>();
    if (n_eff > 0) PX_HIP(px::launch_pq_scan(a, s));
    if (p->timing.enabled) PX_HIP(hipEventRecord(p->timing.ev[1], s));

    px::MergeArgs mg{};
    mg.dbg = p->ws.dbg;
    mg.part_keys = a.part_keys;
    mg.part_ids = a.part_ids;
    mg.rowidx = rowidx;
    mg.width = n_eff > 0 ? (int)width : 0;
    mg.nq = (int)nq;
    mg.kl = kl;
    mg.k = (int)k;
    mg.metric = p->metric;
    mg.corpus = nullptr;  // ADC keys are already the reference's
    mg.sorted_lists = 1;
    mg.out_ids = d_ids;
    mg.out_dists = d_out;
    mg.raw_keys = 0;
    PX_HIP(px::launch_merge(mg, s));
    if (p->timing.enabled) PX_HIP(hipEventRecord(p->timing.ev[2], s));
    PX_HIP(hipStreamSynchronize(s));
    if (p->timing.enabled) {
        PX_HIP(hipEventElapsedTime(&p->timing.scan_ms, p->timing.ev[0], p->timing.ev[1]));
        PX_HIP(hipEventElapsedTime(&p->timing.total_ms, p->timing.ev[0], p->timing.ev[2]));
        p->timing.splits = splits;
        p->timing.blocks = (int)(groups * splits);
    }
    return PX_OK;
}

}  // namespace

// ---------------------------------------------------------------------------------------
// Fixed scratch of px_flat_search_device_noalloc: the entry point for callers that cannot
// allocate device memory. Each GPU the library runs on holds its own copy of this array
// from the code object's load until the process ends. In host code `scratch` names a
// host-side stand-in, not device memory: every use goes through the device address that
// hipGetSymbolAddress returns for the device.
// ---------------------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
// Largest k the entry point serves (its k + 8 candidates fit the per-split lists).
constexpr int64_t kNoAllocMaxK = px::kMaxList - kReRankMargin;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
constexpr int kMaxScratchDevices = 64;
unsigned char* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on `device`, looked up once per device with that device
// current (the caller has made it current).
int scratch_of_device(int device, unsigned char** out) {
    if (device < 0 || device >= kMaxScratchDevices)
        return fail(PX_ERR_DEVICE, "device ordinal out of range for the fixed scratch");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(e != hipSuccess ? (int)e : PX_ERR_DEVICE,
                        std::string("hipGetSymbolAddress of the fixed scratch failed: ") +
                            hipGetErrorString(e));
        g_scratch_ptr[device] = static_cast<unsigned char*>(ptr);
    }
    *out = g_scratch_ptr[device];
    return PX_OK;
}

// Bump layout over the fixed scratch: 256-byte aligned pieces in order. With base ==
// nullptr it only measures.
struct ScratchLayout {
    unsigned char* base = nullptr;
    size_t used = 0;
    template <class T>
    T* take(size_t count) {
        const size_t off = (used + 255) / 256 * 256;
        used = off + count * sizeof(T);
        return base ? reinterpret_cast<T*>(base + off) : nullptr;
    }
};

}  // namespace


// ---------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------
extern "C" {

const char* px_last_error(void) { return g_err.c_str(); }
const char* px_version(void) { return "0.1.0"; }

int px_flat_create(int metric, int64_t dim, px_flat** out) {
    if (!out) return fail(PX_ERR_ARG, "null output handle pointer");
    *out = nullptr;
    if (metric != 0 && metric != 1) return fail(PX_ERR_ARG, "metric must be 0 (L2) or 1 (InnerProduct)");
    if (dim <= 0) return fail(PX_ERR_DIM, "dim must be > 0");
    px_flat* f = new (std::nothrow) px_flat();
    if (!f) return fail(PX_ERR_ARG, "out of host memory");
    f->metric = metric;
    f->smetric = metric;
    f->dim = dim;
    f->dp = px::padded_dim(dim);
    *out = f;
    return PX_OK;
}

void px_flat_destroy(px_flat* f) {
    if (!f) return;
    if (f->dev.device >= 0) {
        (void)hipSetDevice(f->dev.device);
        if (f->stream) (void)hipStreamSynchronize(f->stream);
        dev_free(f->d_x);
        dev_free(f->d_norm);
        dev_free(f->d_xh);
        f->ws.release();
        f->timing.destroy();
        if (f->stream) (void)hipStreamDestroy(f->stream);
    }
    delete f;
}

int px_flat_add(px_flat* f, const float* vectors, int64_t n) {
    if (!f) return fail(PX_ERR_ARG, "null index handle");
    if (n < 0 || (n > 0 && !vectors)) return fail(PX_ERR_ARG, "bad vectors pointer or count");
    if (n == 0) return PX_OK;
    if (!all_finite(vectors, n * f->dim))
        return fail(PX_ERR_NONFINITE, "vectors must not contain NaN or infinite values");
    if (f->n + n > (int64_t)INT32_MAX - 1)
        return fail(PX_ERR_ARG, "index would exceed 2^31 - 2 rows");
    std::lock_guard<std::mutex> lock(f->mu);
    // the rows count only once they are mirrored: a failed upload (e.g. out of device
    // memory) leaves the index as it was, as the reference's add either completes or panics
    const size_t pending0 = f->pending.size();
    const int64_t n0 = f->n;
    f->pending.insert(f->pending.end(), vectors, vectors + n * f->dim);
    f->n += n;
    if (px_device_count() > 0) {
        const int rc = flat_sync(f);
        if (rc != PX_OK) {
            f->pending.resize(pending0);
            f->n = n0;
            return rc;
        }
    }
    return PX_OK;
}

int px_flat_search(const px_flat* cf, const float* queries, int64_t nq, int64_t k,
                   const uint8_t* mask, int64_t* out_ids, float* out_dists) {
    PX_TRY(check_search_args(cf, queries, nq, k, out_ids, out_dists));
    // crates/py/src/lib.rs:127-128 validates the queries before the k == 0 early return (a
    // search proper checks them in flat_search_host, in the same pass as their fp16 test)
    if (k == 0 || nq == 0) {
        if (queries && !all_finite(queries, nq * cf->dim))
            return fail(PX_ERR_NONFINITE, "query must not contain NaN or infinite values");
        return PX_OK;
    }
    return flat_search_host(const_cast<px_flat*>(cf), cf->metric, queries, nq, k, mask, out_ids,
                            out_dists, 0);
}

int px_flat_search_device(const px_flat* cf, const float* d_queries, int64_t nq, int64_t k,
                          const uint8_t* d_mask, int64_t* d_ids, float* d_dists) {
    PX_TRY(check_search_args(cf, d_queries, nq, k, d_ids, d_dists));
    if (k == 0 || nq == 0) return PX_OK;
    px_flat* f = const_cast<px_flat*>(cf);
    std::lock_guard<std::mutex> lock(f->mu);
    f->smetric = f->metric;
    PX_TRY(flat_bind(f));
    PX_TRY(flat_sync(f));
    const PendingCheck chk{d_queries, nq * f->dim};
    const float* q = d_queries;
    if (f->dp != f->dim) {
        PX_TRY(f->ws.q.reserve(sizeof(float) * nq * f->dp));
        PX_HIP(px::launch_pad_rows(d_queries, nq, (int)f->dim, (int)f->dp, f->ws.q.as<float>(), f->stream));
        q = f->ws.q.as<float>();
    }
    return flat_run(f, q, nq, k, f->d_rows ? d_mask : nullptr, d_ids, d_dists, 0, &chk);
}

int px_flat_search_device_noalloc(const px_flat* cf, const float* d_queries, int64_t nq,
                                  int64_t k, const uint8_t* d_mask, int64_t* d_ids,
                                  float* d_dists) {
    PX_TRY(check_search_args(cf, d_queries, nq, k, d_ids, d_dists));
    if (k == 0 || nq == 0) return PX_OK;
    if (k > kNoAllocMaxK)
        return fail(PX_ERR_BAD_K, "px_flat_search_device_noalloc serves k <= " +
                                      std::to_string(kNoAllocMaxK) + ", got " + std::to_string(k));
    if (nq > INT32_MAX) return fail(PX_ERR_ARG, "nq must fit 32 bits");
    px_flat* f = const_cast<px_flat*>(cf);
    std::lock_guard<std::mutex> lock(f->mu);
    // binding a device and uploading rows allocate: both must have happened already, in
    // px_flat_add with the device present
    if (f->dev.device < 0 || !f->stream || !f->pending.empty())
        return fail(PX_ERR_DEVICE, "px_flat_search_device_noalloc needs the rows on the device "
                                   "already (px_flat_add with the GPU present)");
    PX_HIP(hipSetDevice(f->dev.device));
    unsigned char* base = nullptr;
    PX_TRY(scratch_of_device(f->dev.device, &base));
    f->smetric = f->metric;
    const int64_t n = f->d_rows;
    const bool masked = d_mask != nullptr && n > 0;
    const int kl = (int)(k + kReRankMargin);
    const bool pad = f->dp != f->dim;
    hipStream_t s = f->stream;

    // the fixed pieces, then the split lists in what remains
    auto fixed = [&](ScratchLayout& L, int** flag, float** q, int** rowidx, int** cscr,
                     int** gtau, int** gbest) {
        *flag = L.take<int>(3);  // finiteness, kept count, the scan's give-up word
        *q = pad ? L.take<float>((size_t)(nq * f->dp)) : nullptr;
        *rowidx = masked ? L.take<int>((size_t)n) : nullptr;
        *cscr = masked ? L.take<int>((size_t)px::mask_compact_scratch(n)) : nullptr;
        *gtau = L.take<int>((size_t)nq);
        *gbest = L.take<int>((size_t)nq * 32);
    };
    ScratchLayout L;
    int *flag, *rowidx, *cscr, *gtau, *gbest;
    float* q;
    fixed(L, &flag, &q, &rowidx, &cscr, &gtau, &gbest);
    const size_t per_split = (size_t)nq * kl * 8 + 512;  // both list arrays, alignment
    if (L.used + per_split > kNoAllocScratchBytes)
        return fail(PX_ERR_ARG, "px_flat_search_device_noalloc: nq=" + std::to_string(nq) +
                                    ", k=" + std::to_string(k) + " need " +
                                    std::to_string(L.used + per_split) +
                                    " bytes of scratch, more than its " +
                                    std::to_string(kNoAllocScratchBytes) + "-byte limit");
    L = ScratchLayout{base, 0};
    fixed(L, &flag, &q, &rowidx, &cscr, &gtau, &gbest);
    const int64_t max_splits = (int64_t)((kNoAllocScratchBytes - L.used) / per_split);

    int h = 0;  // read-backs land in this thread's own memory (no pinned buffer)
    PX_TRY(check_finite_into(d_queries, nq * f->dim, flag, &h, nullptr, s));
    const float* dq = d_queries;
    if (pad) {
        PX_HIP(px::launch_pad_rows(d_queries, nq, (int)f->dim, (int)f->dp, q, s));
        dq = q;
    }
    int64_t n_eff = n;
    if (masked)
        PX_TRY(compact_mask_into(d_mask, n, rowidx, cscr, flag + 1, &h, nullptr, s, &n_eff));
    ListPlan lp;
    PX_TRY(plan_list_scan(n_eff, nq, kl, f->dp, f->dev.cus, &lp, k, max_splits));
    ListBufs b{L.take<float>((size_t)(nq * lp.splits * kl)), nullptr, gtau, gbest, flag + 2,
               nullptr, nullptr};
    b.part_i = L.take<int>((size_t)(nq * lp.splits * kl));
    if (L.used > kNoAllocScratchBytes)
        return fail(PX_ERR_ARG, "internal: scratch layout past its end");  // unreachable
    f->last_rounds = 0;
    f->last_path = PX_PATH_LISTS;
    return flat_run_lists(f, dq, nq, k, n_eff, masked ? rowidx : nullptr, lp, kl, b, d_ids,
                          d_dists, 0, false);
}

int px_flat_get_vectors(const px_flat* cf, int64_t first, int64_t n, float* out) {
    if (!cf || (n > 0 && !out)) return fail(PX_ERR_ARG, "null argument");
    if (first < 0 || n < 0 || first + n > cf->n) return fail(PX_ERR_ARG, "row range out of bounds");
    if (n == 0) return PX_OK;
    px_flat* f = const_cast<px_flat*>(cf);
    std::lock_guard<std::mutex> lock(f->mu);
    // rows [0, d_rows) live in HBM (padded pitch), the rest in the host pending buffer
    const int64_t dev_hi = std::min(first + n, f->d_rows);
    if (first < dev_hi) {
        PX_TRY(flat_bind(f));
        if (f->dp == f->dim) {
            PX_HIP(hipMemcpyAsync(out, f->d_x + first * f->dp, sizeof(float) * (dev_hi - first) * f->dp,
                                  hipMemcpyDeviceToHost, f->stream));
            PX_HIP(hipStreamSynchronize(f->stream));
        } else {
            // padded rows come down contiguously in 64 MB chunks (a pitched copy to host
            // memory is staged row by row) and drop their pad columns on the host
            const int64_t chunk =
                std::max<int64_t>(1, ((int64_t)64 << 20) / ((int64_t)sizeof(float) * f->dp));
            std::vector<float> stage((size_t)(std::min(chunk, dev_hi - first) * f->dp));
            for (int64_t r = first; r < dev_hi; r += chunk) {
                const int64_t nr = std::min(chunk, dev_hi - r);
                PX_HIP(hipMemcpyAsync(stage.data(), f->d_x + r * f->dp, sizeof(float) * nr * f->dp,
                                      hipMemcpyDeviceToHost, f->stream));
                PX_HIP(hipStreamSynchronize(f->stream));
                for (int64_t i = 0; i < nr; ++i)
                    std::memcpy(out + (r - first + i) * f->dim, stage.data() + i * f->dp,
                                sizeof(float) * f->dim);
            }
        }
    }
    for (int64_t r = std::max(first, f->d_rows); r < first + n; ++r)
        std::memcpy(out + (r - first) * f->dim, f->pending.data() + (r - f->d_rows) * f->dim,
                    sizeof(float) * f->dim);
    return PX_OK;
}

int64_t px_flat_size(const px_flat* f) { return f ? f->n : 0; }
int64_t px_flat_dim(const px_flat* f) { return f ? f->dim : 0; }
int px_flat_metric(const px_flat* f) { return f ? f->metric : -1; }
int64_t px_flat_memory_bytes(const px_flat* f) {
    return f ? f->n * f->dim * (int64_t)sizeof(float) : 0;
}

int px_flat_set_timing(px_flat* f, int enable) {
    if (!f) return fail(PX_ERR_ARG, "null index handle");
    f->timing.enabled = enable != 0;
    return PX_OK;
}

int px_flat_last_timing(const px_flat* f, float* scan_ms, float* total_ms, int* splits,
                        int* blocks) {
    if (!f) return fail(PX_ERR_ARG, "null index handle");
    if (scan_ms) *scan_ms = f->timing.scan_ms;
    if (total_ms) *total_ms = f->timing.total_ms;
    if (splits) *splits = f->timing.splits;
    if (blocks) *blocks = f->timing.blocks;
    return PX_OK;
}

int px_flat_last_rounds(const px_flat* f, int* rounds) {
    if (!f) return fail(PX_ERR_ARG, "null index handle");
    if (rounds) *rounds = f->last_rounds;
    return PX_OK;
}

int px_flat_set_scan_f16(px_flat* f, int enable) {
    if (!f) return fail(PX_ERR_ARG, "null index handle");
    std::lock_guard<std::mutex> lock(f->mu);
    f->scan_f16 = enable != 0;
    return PX_OK;
}

int px_flat_set_spin_limit(px_flat* f, int polls) {
    if (!f) return fail(PX_ERR_ARG, "null index handle");
    if (polls < 0) return fail(PX_ERR_ARG, "spin limit must be >= 0");
    std::lock_guard<std::mutex> lock(f->mu);
    f->spin_limit = polls;
    return PX_OK;
}

int px_flat_last_scan_f16(const px_flat* f, int* used) {
    if (!f || !used) return fail(PX_ERR_ARG, "null index handle or output pointer");
    *used = f->last_f16 ? 1 : 0;
    return PX_OK;
}

int px_flat_last_path(const px_flat* f, int* path) {
    if (!f) return fail(PX_ERR_ARG, "null index handle");
    if (path) *path = f->last_path;
    return PX_OK;
}

int px_pq_last_rounds(const px_pq* p, int* rounds) {
    if (!p) return fail(PX_ERR_ARG, "null index handle");
    if (rounds) *rounds = p->last_rounds;
    return PX_OK;
}

// ---- reference GPU seam (gpu.rs:10-15) ------------------------------------------------
PxGpuIndex* knn_gpu_create(const float* base, int n, int dim) {
    if (!base || n < 0 || dim <= 0) return nullptr;
    PxGpuIndex* g = new (std::nothrow) PxGpuIndex();
    if (!g) return nullptr;
    // knn.cu:123-141: the corpus is on the device when create returns, else NULL. One copy
    // (rows and squared norms) serves both metrics; knn_gpu_search names the metric per
    // call (knn.cu:143-174). The handle's own metric code is never used.
    if (px_flat_create(0, dim, &g->flat) != PX_OK || px_flat_add(g->flat, base, n) != PX_OK ||
        flat_bind(g->flat) != PX_OK || flat_sync(g->flat) != PX_OK) {
        knn_gpu_free(g);
        return nullptr;
    }
    return g;
}

int knn_gpu_search(const PxGpuIndex* g, const float* queries, int nq, int k, int metric,
                   long long* out_ids, float* out_keys) {
    if (!g) return fail(PX_ERR_ARG, "null index handle");
    if (k < 1 || k > PX_MAX_K) return fail(PX_ERR_BAD_K, "k out of range");  // knn.cu:145
    if (nq <= 0) return PX_OK;
    PX_TRY(check_search_args(g->flat, queries, nq, k, out_ids, out_keys));
    // knn.cu's kernel: metric 0 is L2, anything else the inner product
    return flat_search_host(g->flat, metric == 0 ? 0 : 1, queries, nq, k, nullptr,
                            reinterpret_cast<int64_t*>(out_ids), out_keys, 1);
}

void knn_gpu_free(PxGpuIndex* g) {
    if (!g) return;
    px_flat_destroy(g->flat);
    delete g;
}

// ---- PQ ------------------------------------------------------------------------------
int px_pq_create(int metric, int64_t dim, int64_t m, int64_t nbits, px_pq** out) {
    if (!out) return fail(PX_ERR_ARG, "null output handle pointer");
    *out = nullptr;
    if (metric != 0 && metric != 1) return fail(PX_ERR_ARG, "metric must be 0 (L2) or 1 (InnerProduct)");
    if (m < 1) return fail(PX_ERR_ARG, "m must be >= 1");
    if (dim <= 0 || dim % m != 0) return fail(PX_ERR_DIM, "dim must be > 0 and divisible by m");
    if (nbits < 1 || nbits > 8) return fail(PX_ERR_ARG, "nbits must be in 1..=8");
    px_pq* p = new (std::nothrow) px_pq();
    if (!p) return fail(PX_ERR_ARG, "out of host memory");
    p->metric = metric;
    p->dim = dim;
    p->m = m;
    p->nbits = nbits;
    p->ks = (int64_t)1 << nbits;
    p->dsub = dim / m;
    *out = p;
    return PX_OK;
}

void px_pq_destroy(px_pq* p) {
    if (!p) return;
    if (p->dev.device >= 0) {
        (void)hipSetDevice(p->dev.device);
        if (p->stream) (void)hipStreamSynchronize(p->stream);
        dev_free(p->d_books);
        dev_free(p->d_codes);
        p->ws.release();
        p->timing.destroy();
        if (p->stream) (void)hipStreamDestroy(p->stream);
    }
    delete p;
}

int px_pq_train(px_pq* p, const float* training, int64_t n, int64_t train_iters,
                int64_t train_sample, uint64_t seed) {
    if (!p) return fail(PX_ERR_ARG, "null index handle");
    if (n < 0 || (n > 0 && !training) || train_iters < 0 || train_sample < 0)
        return fail(PX_ERR_ARG, "bad training arguments");
    if (n < p->ks)
        return fail(PX_ERR_ARG, "training set too small: need at least " + std::to_string(p->ks) +
                                    " rows for nbits=" + std::to_string(p->nbits) + ", got " +
                                    std::to_string(n));
    if (!all_finite(training, n * p->dim))
        return fail(PX_ERR_NONFINITE, "training data must not contain NaN or infinite values");
    std::vector<float> books((size_t)(p->m * p->ks * p->dsub));
    std::lock_guard<std::mutex> lock(p->mu);
    // on the GPU when one is present, else on the host (as the reference does); both give
    // the same codebooks bit for bit
    if (px_device_count() > 0)
        PX_TRY(pq_train_device(p, training, n, train_iters, train_sample, seed, books.data()));
    else
        px::pq_train_host(training, n, p->dim, p->m, p->nbits, train_iters, train_sample, seed,
                          books.data());
    p->codebooks.swap(books);
    p->trained = true;
    p->books_on_device = false;
    p->codes.clear();  // PqIndex::train builds a fresh index (pq.rs:226-229)
    p->n = 0;
    p->d_rows = 0;
    return PX_OK;
}

int px_pq_set_codebooks(px_pq* p, const float* codebooks) {
    if (!p || !codebooks) return fail(PX_ERR_ARG, "null argument");
    const size_t len = (size_t)(p->m * p->ks * p->dsub);
    if (!all_finite(codebooks, (int64_t)len))
        return fail(PX_ERR_NONFINITE, "codebooks must not contain NaN or infinite values");
    std::lock_guard<std::mutex> lock(p->mu);
    p->codebooks.assign(codebooks, codebooks + len);
    p->trained = true;
    p->books_on_device = false;
    return PX_OK;
}

int px_pq_get_codebooks(const px_pq* p, float* out) {
    if (!p || !out) return fail(PX_ERR_ARG, "null argument");
    if (!p->trained) return fail(PX_ERR_UNTRAINED, "index is not trained");
    std::memcpy(out, p->codebooks.data(), sizeof(float) * p->codebooks.size());
    return PX_OK;
}

int px_pq_add(px_pq* p, const float* vectors, int64_t n) {
    if (!p) return fail(PX_ERR_ARG, "null index handle");
    if (!p->trained) return fail(PX_ERR_UNTRAINED, "index is not trained; call train() first");
    if (n < 0 || (n > 0 && !vectors)) return fail(PX_ERR_ARG, "bad vectors pointer or count");
    if (n == 0) return PX_OK;
    if (!all_finite(vectors, n * p->dim))
        return fail(PX_ERR_NONFINITE, "vectors must not contain NaN or infinite values");
    std::vector<uint8_t> codes((size_t)(n * p->m));
    if (px_device_count() > 0) {
        std::lock_guard<std::mutex> lock(p->mu);
        PX_TRY(pq_encode_device(p, vectors, n, codes.data()));
    } else {
        px::pq_encode_host(p->codebooks.data(), p->dim, p->m, p->nbits, vectors, n, codes.data());
    }
    return px_pq_add_codes(p, codes.data(), n);
}

int px_pq_add_codes(px_pq* p, const uint8_t* codes, int64_t n) {
    if (!p) return fail(PX_ERR_ARG, "null index handle");
    if (!p->trained) return fail(PX_ERR_UNTRAINED, "index is not trained; call train() first");
    if (n < 0 || (n > 0 && !codes)) return fail(PX_ERR_ARG, "bad codes pointer or count");
    if (n == 0) return PX_OK;
    if (p->n + n > (int64_t)INT32_MAX - 1) return fail(PX_ERR_ARG, "index would exceed 2^31 - 2 rows");
    for (int64_t i = 0; i < n * p->m; ++i)
        if (codes[i] >= p->ks) return fail(PX_ERR_ARG, "code value out of range for nbits");
    std::lock_guard<std::mutex> lock(p->mu);
    // as px_flat_add: the rows count only once they are on the device
    const int64_t n0 = p->n;
    p->codes.insert(p->codes.end(), codes, codes + n * p->m);
    p->n += n;
    if (px_device_count() > 0) {
        const int rc = pq_sync(p);
        if (rc != PX_OK) {
            p->codes.resize((size_t)(n0 * p->m));
            p->n = n0;
            return rc;
        }
    }
    return PX_OK;
}

int px_pq_get_codes(const px_pq* p, int64_t first, int64_t n, uint8_t* out) {
    if (!p || (n > 0 && !out)) return fail(PX_ERR_ARG, "null argument");
    if (first < 0 || n < 0 || first + n > p->n) return fail(PX_ERR_ARG, "code range out of bounds");
    std::memcpy(out, p->codes.data() + first * p->m, (size_t)(n * p->m));
    return PX_OK;
}

int px_pq_search(const px_pq* cp, const float* queries, int64_t nq, int64_t k,
                 const uint8_t* mask, int64_t* out_ids, float* out_dists) {
    PX_TRY(check_search_args(cp, queries, nq, k, out_ids, out_dists));
    px_pq* p = const_cast<px_pq*>(cp);
    if (!p->trained) return fail(PX_ERR_UNTRAINED, "index is not trained");
    if (queries && !all_finite(queries, nq * p->dim))
        return fail(PX_ERR_NONFINITE, "query must not contain NaN or infinite values");
    if (k == 0 || nq == 0) return PX_OK;
    std::lock_guard<std::mutex> lock(p->mu);
    if (p->n == 0) {
        host_padding(p->metric, nq, k, out_ids, out_dists, 0);
        return PX_OK;
    }
    PX_TRY(pq_sync(p));
    Workspace& ws = p->ws;
    hipStream_t s = p->stream;
    const float* d_q = nullptr;
    PX_TRY(upload_queries(ws, queries, nq, p->dim, p->dim, s, &d_q));
    const uint8_t* d_mask = nullptr;
    if (mask) {
        PX_TRY(ws.mask.reserve(p->d_rows));
        PX_HIP(hipMemcpyAsync(ws.mask.p, mask, p->d_rows, hipMemcpyHostToDevice, s));
        d_mask = ws.mask.as<uint8_t>();
    }
    PX_TRY(ws.out_ids.reserve(sizeof(int64_t) * nq * k));
    PX_TRY(ws.out_d.reserve(sizeof(float) * nq * k));
    PX_TRY(pq_run(p, d_q, nq, k, d_mask, ws.out_ids.as<int64_t>(), ws.out_d.as<float>()));
    return download_results(ws, nq, k, s, out_ids, out_dists);
}

int px_pq_search_device(const px_pq* cp, const float* d_queries, int64_t nq, int64_t k,
                        const uint8_t* d_mask, int64_t* d_ids, float* d_dists) {
    PX_TRY(check_search_args(cp, d_queries, nq, k, d_ids, d_dists));
    px_pq* p = const_cast<px_pq*>(cp);
    if (!p->trained) return fail(PX_ERR_UNTRAINED, "index is not trained");
    if (k == 0 || nq == 0) return PX_OK;
    std::lock_guard<std::mutex> lock(p->mu);
    PX_TRY(pq_sync(p));
    PX_TRY(check_device_finite(p->ws, d_queries, nq * p->dim, p->stream));
    return pq_run(p, d_queries, nq, k, p->d_rows ? d_mask : nullptr, d_ids, d_dists);
}

int px_pq_is_trained(const px_pq* p) { return p && p->trained ? 1 : 0; }
int64_t px_pq_size(const px_pq* p) { return p ? p->n : 0; }
int64_t px_pq_dim(const px_pq* p) { return p ? p->dim : 0; }
int64_t px_pq_m(const px_pq* p) { return p ? p->m : 0; }
int64_t px_pq_nbits(const px_pq* p) { return p ? p->nbits : 0; }
int px_pq_metric(const px_pq* p) { return p ? p->metric : -1; }
int64_t px_pq_memory_bytes(const px_pq* p) {
    if (!p || !p->trained) return 0;
    return p->n * p->m + (int64_t)(p->codebooks.size() * sizeof(float));
}
int64_t px_pq_raw_bytes(const px_pq* p) {
    return p && p->trained ? p->n * p->dim * (int64_t)sizeof(float) : 0;
}

int px_pq_set_timing(px_pq* p, int enable) {
    if (!p) return fail(PX_ERR_ARG, "null index handle");
    p->timing.enabled = enable != 0;
    return PX_OK;
}

int px_pq_last_timing(const px_pq* p, float* scan_ms, float* total_ms, int* splits, int* blocks) {
    if (!p) return fail(PX_ERR_ARG, "null index handle");
    if (scan_ms) *scan_ms = p->timing.scan_ms;
    if (total_ms) *total_ms = p->timing.total_ms;
    if (splits) *splits = p->timing.splits;
    if (blocks) *blocks = p->timing.blocks;
    return PX_OK;
}

// ---- device info and plumbing ---------------------------------------------------------
int px_device_count(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) return 0;
    return count;
}

int px_device_info(int device, char* name, size_t name_len, int* cu_count, int64_t* hbm_bytes,
                   int* clock_khz, char* arch, size_t arch_len) {
    if (px_device_count() <= device || device < 0)
        return fail(PX_ERR_DEVICE, "no such HIP device");
    hipDeviceProp_t prop;
    PX_HIP(hipGetDeviceProperties(&prop, device));
    if (name && name_len) {
        std::strncpy(name, prop.name, name_len - 1);
        name[name_len - 1] = 0;
    }
    if (arch && arch_len) {
        std::strncpy(arch, prop.gcnArchName, arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    if (cu_count) *cu_count = prop.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = (int64_t)prop.totalGlobalMem;
    if (clock_khz) *clock_khz = prop.clockRate;
    return PX_OK;
}

int px_hip_versions(int* runtime_version, int* driver_version) {
    int rt = 0, dv = 0;
    PX_HIP(hipRuntimeGetVersion(&rt));
    PX_HIP(hipDriverGetVersion(&dv));
    if (runtime_version) *runtime_version = rt;
    if (driver_version) *driver_version = dv;
    return PX_OK;
}

int px_dev_alloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(PX_ERR_ARG, "null pointer");
    PX_HIP(hipMalloc(ptr, bytes));
    return PX_OK;
}
int px_dev_free(void* ptr) {
    PX_HIP(hipFree(ptr));
    return PX_OK;
}
int px_dev_upload(void* dst, const void* src, size_t bytes) {
    PX_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return PX_OK;
}
int px_dev_download(void* dst, const void* src, size_t bytes) {
    PX_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return PX_OK;
}
int px_dev_copy_kernel(void* dst, const void* src, size_t bytes, float* ms) {
    if (bytes % 16) return fail(PX_ERR_ARG, "bytes must be a multiple of 16");
    hipEvent_t e0, e1;
    PX_HIP(hipEventCreate(&e0));
    PX_HIP(hipEventCreate(&e1));
    PX_HIP(hipEventRecord(e0, nullptr));
    PX_HIP(px::launch_copy(static_cast<const float4*>(src), static_cast<float4*>(dst),
                           (int64_t)(bytes / 16), nullptr));
    PX_HIP(hipEventRecord(e1, nullptr));
    PX_HIP(hipEventSynchronize(e1));
    float t = 0.f;
    PX_HIP(hipEventElapsedTime(&t, e0, e1));
    if (ms) *ms = t;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return PX_OK;
}

int px_dev_lds_gather(int random, int blocks, int iters, float* ms, double* bytes) {
    if (blocks <= 0 || iters <= 0) return fail(PX_ERR_ARG, "blocks and iters must be positive");
    const int nt = px::lds_gather_threads();
    float* out = nullptr;
    PX_HIP(dev_malloc(&out, sizeof(float) * (size_t)blocks * nt));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    float t = 0.f;
    if (e == hipSuccess) e = hipEventRecord(e0, nullptr);
    if (e == hipSuccess) e = px::launch_lds_gather(random, blocks, iters, out, nullptr);
    if (e == hipSuccess) e = hipEventRecord(e1, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    dev_free(out);
    PX_HIP(e);
    if (ms) *ms = t;
    if (bytes) *bytes = (double)blocks * nt * iters * 16.0 * 16.0;
    return PX_OK;
}

}  // extern "C"
