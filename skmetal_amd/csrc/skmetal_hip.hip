// skmetal_hip.hip -- host runtime and C ABI of libskmetal_hip.so.
//
// Replaces the reference's Swift bridge on the KMeans path
// (skmetal_bridge/Sources/SkMetalBridge/{MetalContext,Bridge,KMeansBridge}.swift):
//   - MetalContext.shared (device, queue, buffer pool)  -> Context below
//   - makeBuffer(bytesNoCopy:) zero-copy wrapping       -> hipMalloc'd device
//     buffers, filled through pinned staging with hipMemcpyAsync; X stays
//     resident in HBM for the whole fit
//   - one command buffer + waitUntilCompleted per Lloyd iteration
//     (KMeansBridge.swift:249-313)                      -> all iterations of a
//     batch enqueued on one stream; kernels read a device-side `done` flag
//     and return at once after the loop has stopped, so the host synchronises
//     once per batch, not once per iteration.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include <dlfcn.h>
#include <rocblas/rocblas.h>  // types only: librocblas is opened on the first skmetal_gemm

#include "skmetal_hip.h"
#include "internal.h"

using namespace skm;

// Device memory of skmetal_hip_kmeans_batch_fused_noalloc: every buffer that
// entry point needs besides its inputs and outputs is carved from this array,
// one copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel: it uses the device address taken once per device
// with hipGetSymbolAddress at initialisation (scratch_address below).
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch_addr[kMaxDevices] = {};  // device address of `scratch`, per device id (guarded by the context lock)
constexpr long kNoAllocMaxRows = long(1) << 22;  // rows the scratch holds relocation distances for


thread_local std::string g_err;

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    int code = SKMETAL_EHIP;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) code = SKMETAL_ENOMEM;
    if (e == hipErrorLaunchFailure || e == hipErrorInvalidDeviceFunction || e == hipErrorLaunchOutOfResources)
        code = SKMETAL_ELAUNCH;
    return fail(code, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                       \
    do {                                          \
        hipError_t e_ = (expr);                   \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

#define TRY(expr)                \
    do {                         \
        int rc_ = (expr);        \
        if (rc_ != 0) return rc_; \
    } while (0)

// The device address of `scratch` on device `dev` (current), taken once.
int scratch_address(int dev, void** out)
{
    if (dev < 0 || dev >= kMaxDevices) return fail(SKMETAL_ERANGE, "device id %d out of range", dev);
    if (g_scratch_addr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return fail(SKMETAL_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return 0;
}

constexpr size_t kPinBytes = size_t(32) << 20;  // per staging buffer
// finalize in record mode (sorted update): sized as for 128 partials, i.e.
// 16 columns x 16 lanes per block; a cluster's records are read in batches
constexpr int kRecR = 128;
constexpr size_t kMaxDim = size_t(1) << 20;
constexpr size_t kMaxTimedSteps = 4096;  // steps skmetal_hip_lloyd_iterate can time per kernel

// ---------------------------------------------------------------------------
// context: device, stream, pinned staging, size-keyed device buffer cache
// (the analogue of MetalContext.reusableBuffer/recycleBuffer, :66-85)
// ---------------------------------------------------------------------------
struct Context {
    std::recursive_mutex mu;
    bool ready = false;
    int dev = 0;
    int num_cu = 0;
    int max_threads = 0;
    size_t total_mem = 0;
    std::string name;
    hipStream_t stream = nullptr;
    void* scratch = nullptr;  // device address of this device's `scratch` array
    void* pin[2] = {nullptr, nullptr};
    hipEvent_t pin_ev[2] = {nullptr, nullptr};
    std::multimap<size_t, void*> free_blocks;
    std::map<void*, size_t> sizes;

    int init()
    {
        if (ready) return 0;
        int count = 0;
        hipError_t e = hipGetDeviceCount(&count);
        if (e != hipSuccess || count < 1)
            return fail(SKMETAL_ENODEV, "no HIP device available (%s)", e == hipSuccess ? "0 devices" : hipGetErrorString(e));
        HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
        hipDeviceProp_t p;
        HIP_TRY(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
        if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
            return fail(SKMETAL_ENODEV, "device %d is %s; this library is built for gfx950 (MI355X)", dev,
                        p.gcnArchName);
        num_cu = p.multiProcessorCount;
        max_threads = p.maxThreadsPerBlock;
        total_mem = p.totalGlobalMem;
        name = p.name;
        HIP_TRY(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        TRY(scratch_address(dev, &scratch));
        for (int i = 0; i < 2; ++i) {
            HIP_TRY(hipHostMalloc(&pin[i], kPinBytes, hipHostMallocDefault), "hipHostMalloc(staging)");
            HIP_TRY(hipEventCreateWithFlags(&pin_ev[i], hipEventDisableTiming), "hipEventCreate");
        }
        ready = true;
        return 0;
    }

    int alloc(void** out, size_t bytes)
    {
        if (bytes == 0) bytes = 256;
        bytes = (bytes + 255) & ~size_t(255);
        auto it = free_blocks.lower_bound(bytes);
        if (it != free_blocks.end() && it->first <= bytes + bytes / 4) {
            *out = it->second;
            free_blocks.erase(it);
            return 0;
        }
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            // drop the cache and retry once
            (void)hipGetLastError();  // clear the failed allocation's error
            release_cache();
            e = hipMalloc(&p, bytes);
            if (e != hipSuccess) return hip_fail(e, "hipMalloc");
        }
        sizes[p] = bytes;
        *out = p;
        return 0;
    }

    void release(void* p)
    {
        if (p == nullptr) return;
        auto it = sizes.find(p);
        if (it == sizes.end()) return;
        free_blocks.emplace(it->second, p);
    }

    void release_cache()
    {
        for (auto& kv : free_blocks) {
            sizes.erase(kv.second);
            (void)hipFree(kv.second);
        }
        free_blocks.clear();
    }
};

Context& ctx()
{
    static Context* c = new Context();  // never destroyed: safe at process exit
    return *c;
}

// Host -> device copy of `rows` rows of `cols` floats into rows of stride
// `ld` floats (pad columns zeroed), through the two pinned staging buffers.
// Host rows [0, m) of `cols` floats into the pinned staging buffer with
// stride ld (pad columns zeroed), split over up to 8 host threads for large
// chunks: one thread's memcpy runs at a fraction of the host's memory
// bandwidth, which would otherwise bound the upload.
static void stage_rows(float* p, const float* src, long m, int cols, int ld)
{
    auto part = [&](long r0, long r1) {
        if (ld == cols) {
            std::memcpy(p + r0 * ld, src + r0 * cols, size_t(r1 - r0) * size_t(ld) * sizeof(float));
        } else {
            for (long i = r0; i < r1; ++i) {
                std::memcpy(p + i * ld, src + i * cols, size_t(cols) * sizeof(float));
                std::memset(p + i * ld + cols, 0, size_t(ld - cols) * sizeof(float));
            }
        }
    };
    const size_t bytes = size_t(m) * size_t(ld) * sizeof(float);
    unsigned nt = std::thread::hardware_concurrency();
    nt = nt < 1 ? 1 : nt > 8 ? 8 : nt;
    if (bytes < (size_t(4) << 20) || nt == 1) {
        part(0, m);
        return;
    }
    std::vector<std::thread> th;
    const long per = (m + nt - 1) / nt;
    for (unsigned t = 1; t < nt; ++t) {
        const long r0 = t * per, r1 = std::min<long>(m, r0 + per);
        if (r0 < r1) th.emplace_back(part, r0, r1);
    }
    part(0, std::min<long>(m, per));
    for (auto& x : th) x.join();
}

// numpy's float32 np.var(X, axis=0) of a C-ordered X [n x d] (numpy
// _core/_methods.py _var, ddof 0), the variances scikit-learn's _tolerance
// averages (sklearn/cluster/_kmeans.py:279-287).  numpy reduces axis 0 row by
// row, so each column's sum and sum of squared deviations are fp32 chains in
// row order, and both divisions by the count run in fp64 (an intp count) and
// round to fp32.  Host threads take contiguous column ranges and run those
// chains: two passes over X, no temporary arrays, numpy's bits.
// Columns [c0, c0 + W) of X: numpy's fp32 chains in row order (sum, then the
// squared deviations from the fp32 mean), the W running values in registers.
template <int W>
static void column_variance_block(const float* X, long n, int d, int c0, float* out)
{
#pragma clang fp contract(off)
    float s[W], s2[W], mean[W];
    for (int c = 0; c < W; ++c) s[c] = 0.f;
    for (long r = 0; r < n; ++r) {
        const float* row = X + r * d + c0;
        for (int c = 0; c < W; ++c) s[c] = s[c] + row[c];
    }
    for (int c = 0; c < W; ++c) {
        mean[c] = (float)((double)s[c] / (double)n);
        s2[c] = 0.f;
    }
    for (long r = 0; r < n; ++r) {
        const float* row = X + r * d + c0;
        for (int c = 0; c < W; ++c) {
            const float t = row[c] - mean[c];
            const float t2 = t * t;
            s2[c] = s2[c] + t2;
        }
    }
    for (int c = 0; c < W; ++c) out[c0 + c] = (float)((double)s2[c] / (double)n);
}

static void column_variance_f32(const float* X, long n, int d, float* out)
{
    // a thread's columns in blocks of 16, 8, 4, 2 and 1
    auto work = [X, n, d, out](int c0, int c1) {
        int c = c0;
        for (; c + 16 <= c1; c += 16) column_variance_block<16>(X, n, d, c, out);
        if (c + 8 <= c1) {
            column_variance_block<8>(X, n, d, c, out);
            c += 8;
        }
        if (c + 4 <= c1) {
            column_variance_block<4>(X, n, d, c, out);
            c += 4;
        }
        if (c + 2 <= c1) {
            column_variance_block<2>(X, n, d, c, out);
            c += 2;
        }
        if (c < c1) column_variance_block<1>(X, n, d, c, out);
    };
    unsigned nt = std::thread::hardware_concurrency();
    const unsigned by_cols = unsigned((d + 7) / 8);  // at least 8 columns (32 bytes of a row) per thread
    nt = std::max(1u, std::min({nt, 16u, by_cols}));
    if (size_t(n) * size_t(d) < (size_t(1) << 20)) nt = 1;
    std::vector<std::thread> th;
    const int per = ((d + int(nt) - 1) / int(nt) + 7) / 8 * 8;
    for (unsigned t = 1; t < nt; ++t) {
        const int c0 = int(t) * per, c1 = std::min(d, c0 + per);
        if (c0 < c1) th.emplace_back(work, c0, c1);
    }
    work(0, std::min(d, per));
    for (auto& x : th) x.join();
}

int upload_rows(Context& C, const float* src, long rows, int cols, int ld, float* dst, hipStream_t s)
{
    const size_t row_bytes = size_t(ld) * sizeof(float);
    const long chunk = std::max<long>(1, long(kPinBytes / row_bytes));
    if (row_bytes > kPinBytes) return fail(SKMETAL_ERANGE, "row of %d floats exceeds the staging buffer", ld);
    int b = 0;
    for (long r = 0; r < rows; r += chunk, b ^= 1) {
        const long m = std::min(chunk, rows - r);
        HIP_TRY(hipEventSynchronize(C.pin_ev[b]), "hipEventSynchronize(staging)");
        float* p = static_cast<float*>(C.pin[b]);
        stage_rows(p, src + r * cols, m, cols, ld);
        HIP_TRY(hipMemcpyAsync(dst + r * ld, p, size_t(m) * row_bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync(H2D)");
        HIP_TRY(hipEventRecord(C.pin_ev[b], s), "hipEventRecord");
    }
    return 0;
}

// Device -> host copy of `rows` rows (stride ld on the device) keeping `cols`.
int download_rows(Context& C, const float* src, long rows, int cols, int ld, float* dst, hipStream_t s)
{
    const size_t row_bytes = size_t(ld) * sizeof(float);
    const long chunk = std::max<long>(1, long(kPinBytes / row_bytes));
    for (long r = 0; r < rows; r += chunk) {
        const long m = std::min(chunk, rows - r);
        float* p = static_cast<float*>(C.pin[0]);
        HIP_TRY(hipEventSynchronize(C.pin_ev[0]), "hipEventSynchronize(staging)");
        HIP_TRY(hipEventSynchronize(C.pin_ev[1]), "hipEventSynchronize(staging)");
        HIP_TRY(hipMemcpyAsync(p, src + r * ld, size_t(m) * row_bytes, hipMemcpyDeviceToHost, s), "hipMemcpyAsync(D2H)");
        HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
        if (ld == cols) {
            std::memcpy(dst + r * cols, p, size_t(m) * row_bytes);
        } else {
            for (long i = 0; i < m; ++i) std::memcpy(dst + (r + i) * cols, p + i * ld, size_t(cols) * sizeof(float));
        }
    }
    return 0;
}

// Plain byte copies through staging (labels and small arrays).
int upload_bytes(Context& C, const void* src, size_t bytes, void* dst, hipStream_t s)
{
    const char* sp = static_cast<const char*>(src);
    char* dp = static_cast<char*>(dst);
    int b = 0;
    for (size_t o = 0; o < bytes; o += kPinBytes, b ^= 1) {
        const size_t m = std::min(kPinBytes, bytes - o);
        HIP_TRY(hipEventSynchronize(C.pin_ev[b]), "hipEventSynchronize(staging)");
        std::memcpy(C.pin[b], sp + o, m);
        HIP_TRY(hipMemcpyAsync(dp + o, C.pin[b], m, hipMemcpyHostToDevice, s), "hipMemcpyAsync(H2D)");
        HIP_TRY(hipEventRecord(C.pin_ev[b], s), "hipEventRecord");
    }
    return 0;
}

// dst[0, bytes) = src, split over up to 8 host threads for large copies (as
// stage_rows: one thread's memcpy runs at a fraction of the host's memory
// bandwidth).
static void par_copy(char* dst, const char* src, size_t bytes)
{
    unsigned nt = std::thread::hardware_concurrency();
    nt = nt < 1 ? 1 : nt > 8 ? 8 : nt;
    if (bytes < (size_t(4) << 20) || nt == 1) {
        std::memcpy(dst, src, bytes);
        return;
    }
    const size_t per = (bytes / nt + 63) & ~size_t(63);
    std::vector<std::thread> th;
    for (unsigned t = 1; t < nt; ++t) {
        const size_t o = t * per;
        if (o < bytes) th.emplace_back([=] { std::memcpy(dst + o, src + o, std::min(per, bytes - o)); });
    }
    std::memcpy(dst, src, std::min(per, bytes));
    for (auto& x : th) x.join();
}

// Device -> host copy through the two pinned staging buffers: chunk i + 1
// goes over the bus into one buffer while the host moves chunk i out of the
// other.
int download_bytes(Context& C, const void* src, size_t bytes, void* dst, hipStream_t s)
{
    const char* sp = static_cast<const char*>(src);
    char* dp = static_cast<char*>(dst);
    if (bytes == 0) return 0;
    HIP_TRY(hipEventSynchronize(C.pin_ev[0]), "hipEventSynchronize(staging)");
    HIP_TRY(hipEventSynchronize(C.pin_ev[1]), "hipEventSynchronize(staging)");
    const size_t nch = (bytes + kPinBytes - 1) / kPinBytes;
    auto issue = [&](size_t i) -> int {
        const size_t o = i * kPinBytes, m = std::min(kPinBytes, bytes - o);
        HIP_TRY(hipMemcpyAsync(C.pin[i & 1], sp + o, m, hipMemcpyDeviceToHost, s), "hipMemcpyAsync(D2H)");
        HIP_TRY(hipEventRecord(C.pin_ev[i & 1], s), "hipEventRecord");
        return 0;
    };
    TRY(issue(0));
    for (size_t i = 0; i < nch; ++i) {
        if (i + 1 < nch) TRY(issue(i + 1));  // its buffer's previous chunk (i - 1) is already out
        HIP_TRY(hipEventSynchronize(C.pin_ev[i & 1]), "hipEventSynchronize(staging)");
        const size_t o = i * kPinBytes;
        par_copy(dp + o, static_cast<const char*>(C.pin[i & 1]), std::min(kPinBytes, bytes - o));
    }
    return 0;
}

// ---------------------------------------------------------------------------
// One Lloyd problem resident on the device.
// ---------------------------------------------------------------------------
struct Lloyd {
    Context* C = nullptr;
    long n = 0;
    int d = 0, k = 0, ld = 0;
    hipStream_t s = nullptr;
    float* X = nullptr;
    float* cen[2] = {nullptr, nullptr};
    float* cnorm = nullptr;
    float* mean = nullptr;
    int* labels = nullptr;
    float* psum = nullptr;
    int* pcnt = nullptr;
    double* sums = nullptr;
    int* counts = nullptr;
    double* part = nullptr;
    float* shift_sq = nullptr;
    double* rowpart = nullptr;
    float* rowout = nullptr;
    // split E-step with in-stream relocation (rows of at most 128 floats):
    // ||x||^2 per row (set at load) and the E-step's row minima, for the
    // relocation's candidate search
    float* xnorm = nullptr;
    float* emin = nullptr;
    double* colpart = nullptr;
    LoopState* st = nullptr;
    UpdateGeom ug{};
    SortGeom sg{};          // sorted update (generic path), when it applies
    int* s_hist = nullptr;
    int* s_seg = nullptr;
    int* s_counts = nullptr;
    int* s_start = nullptr;
    int* s_roff = nullptr;
    int* s_rcnt = nullptr;
    int* s_perm = nullptr;
    int* s_slab = nullptr;
    float* s_rec = nullptr;
    int fblocks = 0;        // > 0: fused E-step + sums kernel with this many partials
    // kernels over the exact three-part bf16 split: the fused one (f3cap) and
    // the separate E-step (a3cap) exist for this shape; they run while X is
    // in the split's range (split_on, from xmax = the largest |x| of the
    // loaded X, NaN counted as +inf)
    int f3cap = 0;
    int a3cap = 0;
    bool split_on = false;
    float xmax = 0.f;
    unsigned* absmax = nullptr;
    int cur = 0;            // index of the current centres in cen[]
    bool centred = false;
    std::vector<float> h_mean;
    std::vector<void*> owned;

    // no-allocation mode: buffers are carved from [arena, arena + arena_cap)
    // instead of the context's cache
    char* arena = nullptr;
    size_t arena_cap = 0, arena_used = 0;

    int grab(void** p, size_t bytes)
    {
        if (arena != nullptr) {
            const size_t b = (std::max<size_t>(bytes, 1) + 255) & ~size_t(255);
            if (arena_used + b > arena_cap)
                return fail(SKMETAL_ERANGE, "the problem needs more than the %zu bytes of scratch", arena_cap);
            *p = arena + arena_used;
            arena_used += b;
            return 0;
        }
        TRY(C->alloc(p, bytes));
        owned.push_back(*p);
        return 0;
    }

    // A problem on caller-owned device memory (X [n x d], rows of exactly the
    // fused kernels' stride, used as given; the centres are read from Cdev;
    // labels written to labdev) with every other buffer in the arena.  Only the
    // fused step applies (fused_ld(d, k) == d); set-up and the Lloyd loop
    // allocate nothing.
    int create_noalloc(Context* c, long n_, int d_, int k_, const float* Xdev, float* Cdev, int* labdev)
    {
        C = c;
        n = n_;
        d = d_;
        k = k_;
        ld = d;
        s = C->stream;
        ug = update_geometry(n, d, k, C->num_cu);
        fblocks = fused_blocks(n, ld, k, C->num_cu);
        f3cap = fused3_ready(k, ld);
        a3cap = assign3_ready(d, k) && assign3_image_bytes(k, ld) < (size_t(1) << 31);
        const int chunks = std::max(finalize_col_chunks(d, fblocks), (d + kRelocCW - 1) / kRelocCW);
        const size_t kl = size_t(k) * ld;
        X = const_cast<float*>(Xdev);
        labels = labdev;
        cen[0] = Cdev;
        cur = 0;
        centred = false;
        TRY(grab((void**)&cen[1], kl * sizeof(float)));
        TRY(grab((void**)&cnorm, size_t(k) * sizeof(float)));
        TRY(grab((void**)&psum, size_t(fblocks) * kl * sizeof(float)));
        TRY(grab((void**)&pcnt, size_t(fblocks) * k * sizeof(int)));
        TRY(grab((void**)&sums, kl * sizeof(double)));
        TRY(grab((void**)&counts, size_t(k) * sizeof(int)));
        TRY(grab((void**)&part, size_t(k) * chunks * 2 * sizeof(double)));
        TRY(grab((void**)&shift_sq, size_t(k) * sizeof(float)));
        TRY(grab((void**)&rowpart, size_t(rowdist_grid(n)) * sizeof(double)));
        TRY(grab((void**)&st, sizeof(LoopState)));
        TRY(grab((void**)&absmax, sizeof(unsigned)));
        // relocation of empty clusters (k <= 64: always on the device)
        TRY(grab((void**)&rowout, size_t(n) * sizeof(float)));
        TRY(grab((void**)&r_cand_d, size_t(kRelocCandBlocks) * kMaxReloc * sizeof(float)));
        TRY(grab((void**)&r_cand_i, size_t(kRelocCandBlocks) * kMaxReloc * sizeof(long)));
        TRY(grab((void**)&r_amax, sizeof(int)));
        reloc_inline = inline_relocation_on();
        HIP_TRY(hipMemsetAsync(cen[1], 0, kl * sizeof(float), s), "hipMemsetAsync");
        HIP_TRY(hipMemsetAsync(st, 0, sizeof(LoopState), s), "hipMemsetAsync");
        if (f3cap || a3cap) {
            TRY(measure_xmax());
            split_on = split_range_ok(xmax);
        }
        HIP_TRY(launch_cnorm(cen[0], k, ld, cnorm, s), "cnorm launch");
        return 0;
    }

    int create(Context* c, long n_, int d_, int k_)
    {
        C = c;
        n = n_;
        d = d_;
        k = k_;
        const int lf = fused_ld(d, k);
        ld = lf > 0 ? lf : (d + 3) & ~3;
        s = C->stream;
        ug = update_geometry(n, d, k, C->num_cu);
        fblocks = lf > 0 ? fused_blocks(n, ld, k, C->num_cu) : 0;
        f3cap = fblocks > 0 ? fused3_ready(k, ld) : 0;
        // (k_assign3's centre image is addressed with 32-bit buffer offsets)
        a3cap = assign3_ready(d, k) && assign3_image_bytes(k, ld) < (size_t(1) << 31);
        if (fblocks == 0) sg = sort_geometry(n, d, ld, k);
        const int Rmax = sg.on ? 1 : std::max(ug.R, fblocks);
        const int chunks = std::max({finalize_col_chunks(d, ug.R), fblocks > 0 ? finalize_col_chunks(d, fblocks) : 0,
                                     finalize_col_chunks(d, kRecR)});
        const size_t kl = size_t(k) * ld;
        TRY(grab((void**)&X, size_t(n) * ld * sizeof(float)));
        TRY(grab((void**)&cen[0], kl * sizeof(float)));
        TRY(grab((void**)&cen[1], kl * sizeof(float)));
        TRY(grab((void**)&cnorm, size_t(k) * sizeof(float)));
        TRY(grab((void**)&mean, size_t(ld) * sizeof(float)));
        TRY(grab((void**)&labels, size_t(n) * sizeof(int)));
        TRY(grab((void**)&psum, size_t(Rmax) * kl * sizeof(float)));
        TRY(grab((void**)&pcnt, size_t(Rmax) * k * sizeof(int)));
        TRY(grab((void**)&sums, kl * sizeof(double)));
        TRY(grab((void**)&counts, size_t(k) * sizeof(int)));
        TRY(grab((void**)&part, size_t(k) * chunks * 2 * sizeof(double)));
        TRY(grab((void**)&shift_sq, size_t(k) * sizeof(float)));
        TRY(grab((void**)&rowpart, size_t(rowdist_grid(n)) * sizeof(double)));
        TRY(grab((void**)&colpart, size_t(colsum_grid(n)) * d * sizeof(double)));
        TRY(grab((void**)&st, sizeof(LoopState)));
        TRY(grab((void**)&absmax, sizeof(unsigned)));
        reloc_inline = inline_relocation_on();
        if (reloc_inline) {
            TRY(grab((void**)&rowout, size_t(n) * sizeof(float)));
            TRY(grab((void**)&r_cand_d, size_t(kRelocCandBlocks) * kMaxReloc * sizeof(float)));
            TRY(grab((void**)&r_cand_i, size_t(kRelocCandBlocks) * kMaxReloc * sizeof(long)));
            TRY(grab((void**)&r_amax, sizeof(int)));
            if (f3cap || (fblocks == 0 && a3cap && ld <= 128)) {
                TRY(grab((void**)&xnorm, size_t(n) * sizeof(float)));
                TRY(grab((void**)&emin, size_t(n) * sizeof(float)));
            }
        }
        if (sg.on) {
            TRY(grab((void**)&s_hist, size_t(sg.nw) * k * sizeof(int)));
            TRY(grab((void**)&s_seg, size_t(sg.nseg) * k * sizeof(int)));
            TRY(grab((void**)&s_counts, size_t(k) * sizeof(int)));
            TRY(grab((void**)&s_start, size_t(k) * sizeof(int)));
            TRY(grab((void**)&s_roff, size_t(k) * sizeof(int)));
            TRY(grab((void**)&s_rcnt, size_t(k) * sizeof(int)));
            TRY(grab((void**)&s_perm, size_t(n) * sizeof(int)));
            TRY(grab((void**)&s_slab, size_t(n) * sizeof(int)));
            TRY(grab((void**)&s_rec, size_t(sg.max_records) * ld * sizeof(float)));
        }
        HIP_TRY(hipMemsetAsync(cen[0], 0, kl * sizeof(float), s), "hipMemsetAsync");
        HIP_TRY(hipMemsetAsync(cen[1], 0, kl * sizeof(float), s), "hipMemsetAsync");
        HIP_TRY(hipMemsetAsync(mean, 0, size_t(ld) * sizeof(float), s), "hipMemsetAsync");
        HIP_TRY(hipMemsetAsync(st, 0, sizeof(LoopState), s), "hipMemsetAsync");
        HIP_TRY(hipMemsetAsync(labels, 0, size_t(n) * sizeof(int), s), "hipMemsetAsync");
        h_mean.assign(size_t(ld), 0.f);
        return 0;
    }

    // Per-step kernel timing: when kev_base >= 0, step kev_base + i records
    // kev[4i .. 4i+3] before its E-step (or fused) kernel, after it, after
    // the update kernels and after the finalize.  A step enqueued again
    // (after a halt) records again.
    std::vector<hipEvent_t> kev;
    long kev_base = -1;
    // When set, run_loop records it right after each batch of steps is
    // enqueued (before the state read-back): the end of a timed run.
    hipEvent_t batch_end = nullptr;

    void destroy()
    {
        if (s) (void)hipStreamSynchronize(s);  // teardown: nothing to report to
        for (void* p : owned) C->release(p);
        owned.clear();
        pp_release();
        for (hipEvent_t e : kev) (void)hipEventDestroy(e);
        kev.clear();
    }

    int load_X(const float* host, bool center)
    {
        TRY(upload_rows(*C, host, n, d, ld, X, s));
        centred = center;
        if (center) {
            const int nb = colsum_grid(n);
            HIP_TRY(launch_colsum(X, n, ld, d, colpart, nb, s), "colsum launch");
            HIP_TRY(launch_colmean(colpart, nb, n, d, mean, s), "colmean launch");
            HIP_TRY(launch_center(X, n, ld, d, mean, s), "center launch");
            TRY(download_bytes(*C, mean, size_t(d) * sizeof(float), h_mean.data(), s));
        } else {
            std::fill(h_mean.begin(), h_mean.end(), 0.f);
            HIP_TRY(hipMemsetAsync(mean, 0, size_t(ld) * sizeof(float), s), "hipMemsetAsync");
        }
        xmax_known = false;
        split_on = false;
        if (f3cap || a3cap) {
            TRY(measure_xmax());
            split_on = split_range_ok(xmax);
        }
        if (xnorm != nullptr) HIP_TRY(launch_rownorm(X, n, ld, d, xnorm, s), "rownorm launch");
        return 0;
    }

    // max |x| of the loaded X (NaN counted as +inf) into xmax
    bool xmax_known = false;
    int measure_xmax()
    {
        unsigned bits = 0;
        HIP_TRY(launch_absmax(X, n * (long)ld, absmax, s), "absmax launch");
        TRY(download_bytes(*C, absmax, sizeof(unsigned), &bits, s));
        std::memcpy(&xmax, &bits, sizeof(float));
        xmax_known = true;
        return 0;
    }

    // Centres given in caller coordinates -> device (centred like X).
    int set_centers(const float* host)
    {
        TRY(upload_rows(*C, host, k, d, ld, cen[cur], s));
        if (centred) HIP_TRY(launch_center(cen[cur], k, ld, d, mean, s), "center launch");
        HIP_TRY(launch_cnorm(cen[cur], k, ld, cnorm, s), "cnorm launch");
        return 0;
    }

    int get_centers(float* host)
    {
        TRY(download_rows(*C, cen[cur], k, d, ld, host, s));
        if (centred)
            for (int j = 0; j < k; ++j)
                for (int c = 0; c < d; ++c) host[size_t(j) * d + c] = host[size_t(j) * d + c] + h_mean[c];
        return 0;
    }

    int get_labels(int32_t* host) { return download_bytes(*C, labels, size_t(n) * sizeof(int), host, s); }

    int read_state(LoopState* h)
    {
        HIP_TRY(hipMemcpyAsync(h, st, sizeof(LoopState), hipMemcpyDeviceToHost, s), "hipMemcpyAsync(state)");
        HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
        return 0;
    }

    int write_state(const LoopState& h)
    {
        HIP_TRY(hipMemcpyAsync(st, &h, sizeof(LoopState), hipMemcpyHostToDevice, s), "hipMemcpyAsync(state)");
        HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
        return 0;
    }

    char* a3img = nullptr;  // k_assign3's centre image

    int assign(const float* cents, LoopState* state, int* changed, bool minima = false)
    {
        AssignArgs a{X, n, ld, cents, cnorm, k, labels, state, changed, nullptr};
        if (split_on && a3cap) {
            if (a3img == nullptr) TRY(grab((void**)&a3img, assign3_image_bytes(k, ld)));
            a.img = a3img;
            if (minima) a.emin = emin;
            HIP_TRY(launch_assign3(a, C->num_cu, s), "assign launch");
        } else
            HIP_TRY(launch_assign(a, C->num_cu, s), "assign launch");
        return 0;
    }

    // The final E-step with the inertia of its labels: on the split path one
    // pass over X (k_assign3 adds each row's distance to its new centre into
    // per-block totals, k_rowdist_total adds those), else the E-step and then
    // the row-distance pass.
    int assign_inertia(const float* cents, double* out)
    {
        const long blocks = std::min<long>(C->num_cu, (n + 255) / 256);
        if (split_on && a3cap && blocks <= rowdist_grid(n)) {
            if (a3img == nullptr) TRY(grab((void**)&a3img, assign3_image_bytes(k, ld)));
            AssignArgs a{X, n, ld, cents, cnorm, k, labels, nullptr, nullptr, a3img};
            int nb = 0;
            a.inert = rowpart;
            a.inert_blocks = &nb;
            a.d = d;
            HIP_TRY(launch_assign3(a, C->num_cu, s), "assign launch");
            HIP_TRY(launch_inertia_total(rowpart, nb, st, s), "inertia launch");
            LoopState hs{};
            TRY(read_state(&hs));
            *out = hs.inertia;
            return 0;
        }
        TRY(assign(cents, nullptr, nullptr));
        return inertia(out);
    }

    int update()
    {
        if (sg.on) {
            SortArgs a{X, n, ld, d, labels, k, s_hist, s_seg, s_counts, s_start, s_roff, s_rcnt, s_perm, s_slab, s_rec,
                       st};
            HIP_TRY(launch_sorted_update(a, sg, s), "sorted update launch");
            return 0;
        }
        UpdateArgs u{X, n, ld, d, labels, k, psum, pcnt, st};
        HIP_TRY(launch_update(u, ug, s), "update launch");
        return 0;
    }

    // Fused E-step + sums of iteration `iter`; with decide, its blocks first
    // evaluate the stopping rules of iteration iter - 1.
    int fused_step(int iter = 0, bool decide = false, double tol = 0.0, int flags = 0)
    {
        FusedArgs a{X, n, ld, cen[cur], cnorm, k, labels, psum, pcnt, st, fblocks, &st->chg[iter & 1],
                    decide ? 1 : 0, iter, tol, flags, part, finalize_col_chunks(d, fblocks), counts,
                    &st->chg[(iter + 1) & 1], cnorm, shift_sq};
        a.split = split_on && f3cap ? 1 : 0;
        if (a.split) a.emin = emin;
        HIP_TRY(launch_fused(a, s), "fused launch");
        return 0;
    }

    FinalizeArgs finalize_args(int iter, double tol, int flags)
    {
        const bool recs = fblocks == 0 && sg.on;
        const int R = fblocks > 0 ? fblocks : recs ? kRecR : ug.R;
        return FinalizeArgs{recs ? s_rec : psum, pcnt, R, k, d, ld,
                            recs ? s_roff : nullptr, recs ? s_rcnt : nullptr, recs ? s_counts : nullptr,
                            cen[cur], cen[cur ^ 1], cnorm, sums, counts, part, shift_sq,
                            st, iter, tol, flags, finalize_cols(R), &st->chg[iter & 1], &st->chg[(iter + 1) & 1]};
    }

    // One Lloyd step, old centres cen[cur] -> new centres cen[cur ^ 1].  On
    // the fused path the stopping rules of a step are evaluated by the next
    // step's kernel (decide) or, for the last step of a batch (last), by
    // k_finalize_loop; on the generic path by k_finalize_loop every step.
    int enqueue_step(int iter, double tol, int flags, bool decide, bool last)
    {
        hipEvent_t* ev = nullptr;
        if (kev_base >= 0 && iter >= kev_base && 4 * (iter - kev_base + 1) <= (long)kev.size())
            ev = &kev[4 * (iter - kev_base)];
        if (ev) HIP_TRY(hipEventRecord(ev[0], s), "hipEventRecord");
        if (fblocks > 0) {
            TRY(fused_step(iter, decide, tol, flags));
            if (ev) HIP_TRY(hipEventRecord(ev[1], s), "hipEventRecord");
        } else {
            TRY(assign(cen[cur], st, &st->chg[iter & 1], true));
            if (ev) HIP_TRY(hipEventRecord(ev[1], s), "hipEventRecord");
            TRY(update());
        }
        if (ev) HIP_TRY(hipEventRecord(ev[2], s), "hipEventRecord");
        const FinalizeArgs f = finalize_args(iter, tol, flags);
        InRelocArgs r{X, n, ld, d, k, labels, cen[cur], cen[cur ^ 1], sums, counts, part,
                      finalize_col_chunks(d, f.R), rowout, r_cand_d, r_cand_i, r_amax, st, iter};
        if (emin != nullptr && split_on && (fblocks > 0 ? f3cap : a3cap)) {
            // this step's E-step was k_fused3 or k_assign3, which wrote its row minima
            r.xnorm = xnorm;
            r.emin = emin;
        }
        if (reloc_inline && fblocks > 0 && k <= 64 && 8 * ((k * r.nch + 7) / 8) <= kRelocInlineBlocks) {
            // the fused kernel's presence bits name the empty clusters: one launch
            HIP_TRY(launch_finalize_reloc(f, r, s), "finalize launch");
        } else {
            HIP_TRY(launch_finalize(f, s, false), "finalize launch");
            if (reloc_inline) HIP_TRY(launch_reloc_inline(r, s), "relocation launch");
        }
        if (fblocks == 0 || last) HIP_TRY(launch_finalize_loop(f, s), "finalize launch");
        if (ev) HIP_TRY(hipEventRecord(ev[3], s), "hipEventRecord");
        cur ^= 1;
        return 0;
    }

    // Empty clusters at step t (old centres in cen[old]), on the device: the
    // farthest rows move to the empty clusters, the centres are re-averaged
    // from the fp64 sums and the loop decision is taken again (empty clusters
    // no longer stop it).  hs is the state read at the halt; on return it
    // holds the new decision.
    float* r_cand_d = nullptr;
    long* r_cand_i = nullptr;
    int* r_amax = nullptr;
    // k_reloc after every step (empty clusters relocated in-stream); off:
    // the loop halts on an empty cluster and the host starts the relocation
    // (SKMETAL_HIP_HOST_RELOCATE=1 or SKMETAL_HIP_INLINE_RELOCATE=0)
    bool reloc_inline = false;
    bool inline_relocation_on() const
    {
        const char* h = getenv("SKMETAL_HIP_HOST_RELOCATE");
        const char* i = getenv("SKMETAL_HIP_INLINE_RELOCATE");
        return !((h != nullptr && h[0] == '1') || (i != nullptr && i[0] == '0'));
    }
    int device_relocate(int t, int old, double tol, int flags, LoopState& hs)
    {
        if (rowout == nullptr) TRY(grab((void**)&rowout, size_t(n) * sizeof(float)));
        if (r_cand_d == nullptr) {
            TRY(grab((void**)&r_cand_d, size_t(kRelocCandBlocks) * kMaxReloc * sizeof(float)));
            TRY(grab((void**)&r_cand_i, size_t(kRelocCandBlocks) * kMaxReloc * sizeof(long)));
            TRY(grab((void**)&r_amax, sizeof(int)));
        }
        LoopState w = hs;
        w.done = 0;
        TRY(write_state(w));
        RowDistArgs r{X, n, ld, d, cen[old], k, labels, rowout, rowpart, st};
        HIP_TRY(launch_rowdist(r, s), "rowdist launch");
        RelocArgs ra{X, n, ld, d, k, labels, rowout, r_cand_d, r_cand_i, sums, counts, r_amax,
                     cen[old], cen[old ^ 1], part};
        HIP_TRY(launch_relocate(ra, hs.n_empty, s), "relocate launch");
        cur = old;
        FinalizeArgs f = finalize_args(t, tol, flags);
        f.after_reloc = 1;
        HIP_TRY(launch_finalize_loop(f, s, (d + kRelocCW - 1) / kRelocCW), "finalize launch");
        cur = old ^ 1;
        TRY(read_state(&hs));
        return 0;
    }

    // Empty clusters at step t (old centres in cen[old]): sklearn's relocation
    // (_k_means_common.pyx:167-211), averaging (:274-295) and shift on the host
    // from the device's fp64 sums, then upload the new centres to cen[old^1].
    int host_relocate(int t, int old, double tol, int flags, LoopState& hs)
    {
        const size_t kl = size_t(k) * ld;
        std::vector<double> S(kl);
        std::vector<int> cnt(static_cast<size_t>(k));
        std::vector<int> lab(static_cast<size_t>(n));
        std::vector<float> Cold(kl);
        TRY(download_bytes(*C, sums, kl * sizeof(double), S.data(), s));
        TRY(download_bytes(*C, counts, size_t(k) * sizeof(int), cnt.data(), s));
        TRY(download_bytes(*C, labels, size_t(n) * sizeof(int), lab.data(), s));
        TRY(download_bytes(*C, cen[old], kl * sizeof(float), Cold.data(), s));

        std::vector<int> empties;
        for (int j = 0; j < k; ++j)
            if (cnt[size_t(j)] == 0) empties.push_back(j);
        if (!empties.empty()) {
            // distances of every row to its (old) centre, fp32 direct form
            if (rowout == nullptr) TRY(grab((void**)&rowout, size_t(n) * sizeof(float)));
            RowDistArgs r{X, n, ld, d, cen[old], k, labels, rowout, rowpart, st};
            HIP_TRY(launch_rowdist(r, s), "rowdist launch");
            std::vector<float> dist(static_cast<size_t>(n));
            TRY(download_bytes(*C, rowout, size_t(n) * sizeof(float), dist.data(), s));
            float dmax = 0.f;
            for (float v : dist) dmax = std::max(dmax, v);
            if (dmax > 0.f) {
                const size_t ne = empties.size();
                std::vector<long> idx(static_cast<size_t>(n));
                std::iota(idx.begin(), idx.end(), 0L);
                std::partial_sort(idx.begin(), idx.begin() + ne, idx.end(), [&](long a, long b) {
                    return dist[size_t(a)] > dist[size_t(b)] || (dist[size_t(a)] == dist[size_t(b)] && a < b);
                });
                std::vector<float> xr(static_cast<size_t>(ld));
                for (size_t e = 0; e < ne; ++e) {
                    const int j = empties[e];
                    const long far = idx[e];
                    const int o = lab[size_t(far)];
                    TRY(download_bytes(*C, X + far * ld, size_t(ld) * sizeof(float), xr.data(), s));
                    for (int c = 0; c < d; ++c) {
                        S[size_t(o) * ld + c] -= (double)xr[size_t(c)];
                        S[size_t(j) * ld + c] = (double)xr[size_t(c)];
                    }
                    cnt[size_t(j)] = 1;
                    cnt[size_t(o)] -= 1;
                }
            }
        }
        // _average_centers: heaviest cluster first, then rows in order
        int amax = 0;
        for (int j = 1; j < k; ++j)
            if (cnt[size_t(j)] > cnt[size_t(amax)]) amax = j;
        std::vector<double> cur_rows(S);
        for (int j = 0; j < k; ++j) {
            for (int c = 0; c < d; ++c) {
                double& v = cur_rows[size_t(j) * ld + c];
                if (cnt[size_t(j)] > 0)
                    v = v / (double)cnt[size_t(j)];
                else
                    v = cur_rows[size_t(amax) * ld + c];
            }
        }
        std::vector<float> Cn(kl, 0.f), cn(static_cast<size_t>(k));
        double shift_tot = 0.0;
        float shift_max = 0.f;
        for (int j = 0; j < k; ++j) {
            double sq = 0.0, nr = 0.0;
            for (int c = 0; c < d; ++c) {
                const float v = (float)cur_rows[size_t(j) * ld + c];
                Cn[size_t(j) * ld + c] = v;
                const double df = (double)v - (double)Cold[size_t(j) * ld + c];
                sq += df * df;
                nr += (double)v * (double)v;
            }
            shift_tot += (double)(float)sq;
            shift_max = std::max(shift_max, (float)sq);
            cn[size_t(j)] = (float)nr;
        }
        TRY(upload_bytes(*C, Cn.data(), kl * sizeof(float), cen[old ^ 1], s));
        TRY(upload_bytes(*C, cn.data(), size_t(k) * sizeof(float), cnorm, s));
        int done = 0;
        if ((flags & kStopStrict) && hs.last_changed == 0)
            done = 1;
        else if (shift_rule_stops(flags, tol, shift_tot, shift_max))
            done = 2;
        hs.done = done;
        hs.n_iter = t + 1;
        hs.chg[0] = hs.chg[1] = 0;
        hs.shift_tot = shift_tot;
        hs.halt_iter = t;
        TRY(write_state(hs));
        cur = old ^ 1;
        return 0;
    }

    // Lloyd loop from the current centres.  With fixed != 0 exactly max_iter
    // steps run (no convergence stop); otherwise sklearn's rules apply.
    int run_loop(long max_iter, double tol, int flags, bool fixed, int* n_iter_out, int* done_out)
    {
        if (fixed) {
            flags &= ~kStopStrict;
            tol = -1.0;  // no shift rule: sklearn's `shift <= tol` stops at tol = 0 on a zero shift
        }
        LoopState hs{};
        hs.reloc_iter = -1;
        // the reset is a kernel on the stream: nothing waits for the host
        HIP_TRY(launch_state_reset(st, hs, s), "state reset launch");
        HIP_TRY(hipMemsetAsync(labels, 0xff, size_t(n) * sizeof(int), s), "hipMemsetAsync(labels)");
        long it = 0;
        // Steps are enqueued in growing batches and the loop state is read
        // back after each: a halt (convergence, or more empty clusters than
        // k_reloc takes, which the host relocates) then skips at most one
        // batch of launches.  A fixed-iteration run has no convergence stop:
        // with the relocation in-stream it is one batch.
        long batch = fixed ? (reloc_inline ? max_iter : 8) : 4;
        int final_done = 0;
        while (it < max_iter) {
            const long nb = std::min(batch, max_iter - it);
            const int c0 = cur;
            for (long t = it; t < it + nb; ++t) TRY(enqueue_step((int)t, tol, flags, t > it, t + 1 == it + nb));
            if (batch_end) HIP_TRY(hipEventRecord(batch_end, s), "hipEventRecord");
            TRY(read_state(&hs));
            if (hs.done == 3) {
                const int t = hs.halt_iter;
                const int old = (c0 + (t - (int)it)) & 1;
                // SKMETAL_HIP_HOST_RELOCATE=1 keeps the host path (A/B checks)
                const char* env = getenv("SKMETAL_HIP_HOST_RELOCATE");
                const bool on_host =
                    arena == nullptr && ((env != nullptr && env[0] == '1') || hs.n_empty < 1 || hs.n_empty > kMaxReloc);
                if (on_host)
                    TRY(host_relocate(t, old, tol, flags, hs));
                else
                    TRY(device_relocate(t, old, tol, flags, hs));
                if (batch_end) HIP_TRY(hipEventRecord(batch_end, s), "hipEventRecord");
                it = t + 1;
                if (hs.done != 0) {
                    final_done = hs.done;
                    break;
                }
                continue;
            }
            if (hs.done != 0) {
                cur = (c0 + (hs.halt_iter - (int)it) + 1) & 1;
                final_done = hs.done;
                break;
            }
            it += nb;
            batch = std::min<long>(batch * 2, fixed ? 1024 : 64);
        }
        if (n_iter_out) *n_iter_out = max_iter > 0 ? hs.n_iter : 0;
        if (done_out) *done_out = final_done;
        return 0;
    }

    int inertia(double* out)
    {
        RowDistArgs r{X, n, ld, d, cen[cur], k, labels, nullptr, rowpart, st};
        HIP_TRY(launch_rowdist(r, s), "rowdist launch");
        LoopState hs{};
        TRY(read_state(&hs));
        *out = hs.inertia;
        return 0;
    }

    // Greedy k-means++ on the resident X (sklearn's _kmeans_plusplus,
    // _kmeans.py:174-260, unit weights): T candidates per centre after the
    // first, first = the first centre's row, U = the (k - 1) x T uniforms in
    // draw order.  The chosen rows become the current centres; idx_out
    // receives their row indices.  Buffers are kept for further calls.
    PPArgs pp{};
    std::vector<void*> pp_owned;
    int pp_T = 0;

    int pp_grab(void** p, size_t bytes)
    {
        TRY(C->alloc(p, bytes));
        pp_owned.push_back(*p);
        return 0;
    }

    void pp_release()
    {
        for (void* p : pp_owned) C->release(p);
        pp_owned.clear();
        pp_T = 0;
    }

    int plusplus(int T, long first, const double* U, long* idx_out)
    {
        if (T < 1 || T > kPPMaxTrials) return fail(SKMETAL_ERANGE, "n_local_trials=%d not in [1, %d]", T, kPPMaxTrials);
        if (first < 0 || first >= n) return fail(SKMETAL_EINVAL, "first index %ld not in [0, %ld)", first, n);
        if (k > 1 && U == nullptr) return fail(SKMETAL_EINVAL, "null uniforms");
        if (n >= (1L << 31)) return fail(SKMETAL_ERANGE, "k-means++ seeding supports n < 2^31 rows (n=%ld)", n);
        const int nb = (int)((n + kPPRows - 1) / kPPRows);
        if (T != pp_T) {
            pp_release();
            for (int i = 0; i < 2; ++i) {
                TRY(pp_grab((void**)&pp.D[i], size_t(T) * n * sizeof(float)));
                TRY(pp_grab((void**)&pp.P[i], size_t(T) * nb * sizeof(double)));
            }
            TRY(pp_grab((void**)&pp.pfx, size_t(nb) * sizeof(double)));
            TRY(pp_grab((void**)&pp.cand, size_t(T) * sizeof(long)));
            TRY(pp_grab((void**)&pp.idx, size_t(k) * sizeof(long)));
            TRY(pp_grab((void**)&pp.best, size_t(k) * sizeof(int)));
            TRY(pp_grab((void**)&pp.pot, size_t(k) * sizeof(double)));
            TRY(pp_grab((void**)&pp.U, std::max<size_t>(1, size_t(k - 1) * T) * sizeof(double)));
            pp.ctab = nullptr;
            pp.xxn = nullptr;
            if (pp_rows_path(T, ld)) {
                TRY(pp_grab((void**)&pp.ctab, size_t(T) * ld * sizeof(double)));
                TRY(pp_grab((void**)&pp.xxn, size_t(n) * sizeof(double)));
            }
            pp_T = T;
        }
        pp.X = X;
        pp.n = n;
        pp.ld = ld;
        pp.k = k;
        pp.T = T;
        pp.nb = nb;
        pp.cus = C->num_cu;
        pp.centers = cen[cur];
        TRY(upload_bytes(*C, &first, sizeof(long), pp.cand, s));
        if (k > 1) TRY(upload_bytes(*C, U, size_t(k - 1) * T * sizeof(double), const_cast<double*>(pp.U), s));
        HIP_TRY(launch_pp_dist(pp, 0, s), "pp dist launch");
        for (int c = 1; c < k; ++c) {
            HIP_TRY(launch_pp_select(pp, c, s), "pp select launch");
            HIP_TRY(launch_pp_dist(pp, c, s), "pp dist launch");
        }
        HIP_TRY(launch_pp_select(pp, k, s), "pp select launch");
        HIP_TRY(launch_cnorm(cen[cur], k, ld, cnorm, s), "cnorm launch");
        TRY(download_bytes(*C, pp.idx, size_t(k) * sizeof(long), idx_out, s));
        return 0;
    }

    // k-means|| rounds (skmetal's MetalKMeans._kmeans_parallel_init): the
    // squared distance of every row to its nearest candidate so far, kept on
    // the device and lowered with each round's new candidate rows (reset
    // starts it from +inf).  Distances are sklearn's fp32 form, as k-means++'s.
    float* kp_mind = nullptr;
    long* kp_cand = nullptr;
    double* kp_ctab = nullptr;  // [cap16 ld] the candidates' values as fp64 MFMA fragments (rows of <= 128 floats)
    double* kp_ccn = nullptr;   // [cap16] their ||c||^2 (cap16: cap rounded up to a multiple of 16)
    long kp_cap = 0;
    bool kp_valid = false;

    int mindists(const long* rows, long m, int reset, float* out)
    {
        if (n >= (1L << 31)) return fail(SKMETAL_ERANGE, "k-means|| rounds support n < 2^31 rows (n=%ld)", n);
        if (m < 0 || m > (1L << 30)) return fail(SKMETAL_ERANGE, "m=%ld candidate rows out of range", m);
        if (m > 0 && rows == nullptr) return fail(SKMETAL_EINVAL, "null candidate rows");
        if (!reset && !kp_valid) return fail(SKMETAL_EINVAL, "the first k-means|| round must reset the distances");
        for (long i = 0; i < m; ++i)
            if (rows[i] < 0 || rows[i] >= n) return fail(SKMETAL_EINVAL, "candidate row %ld not in [0, %ld)", rows[i], n);
        if (kp_mind == nullptr) TRY(grab((void**)&kp_mind, size_t(n) * sizeof(float)));
        if (m > kp_cap) {
            const long cap = std::max<long>(m, 2 * kp_cap);
            for (void** p : {(void**)&kp_cand, (void**)&kp_ctab, (void**)&kp_ccn})
                if (*p != nullptr) {
                    const auto it = std::find(owned.begin(), owned.end(), *p);
                    if (it != owned.end()) owned.erase(it);
                    C->release(*p);
                    *p = nullptr;
                }
            TRY(grab((void**)&kp_cand, size_t(cap) * sizeof(long)));
            if (pp_rows_min_path(ld)) {  // candidates rounded up to a multiple of 16
                const size_t capp = size_t(cap + 15) / 16 * 16;
                TRY(grab((void**)&kp_ctab, capp * ld * sizeof(double)));
                TRY(grab((void**)&kp_ccn, capp * sizeof(double)));
            }
            kp_cap = cap;
        }
        if (m > 0 || reset) {
            PPArgs a{};
            a.X = X;
            a.n = n;
            a.ld = ld;
            a.nb = (int)((n + kPPRows - 1) / kPPRows);
            a.cand = kp_cand;
            a.mind = kp_mind;
            a.mind_reset = reset ? 1 : 0;
            a.cus = C->num_cu;
            a.ctab = kp_ctab;
            a.ccn = kp_ccn;
            if (m > 0) TRY(upload_bytes(*C, rows, size_t(m) * sizeof(long), kp_cand, s));
            HIP_TRY(launch_pp_mindist(a, (int)m, s), "mindist launch");
        }
        kp_valid = true;
        if (out != nullptr) TRY(download_bytes(*C, kp_mind, size_t(n) * sizeof(float), out, s));
        return 0;
    }

    // numpy's RandomState.choice(n, size, replace=False, p=w / w.sum()) on
    // the device: sample_prepare forms p from the weights (0: the k-means||
    // distances floored at 1e-30, 1: unit weights), sample_draw runs one of
    // choice's passes for the caller's uniforms.
    WSArgs ws{};
    bool ws_ready = false;
    long ws_mcap = 0;

    int sample_prepare(int weights, double* psum, long long* nnz)
    {
        if (weights != 0 && weights != 1) return fail(SKMETAL_EINVAL, "weights=%d is not 0 or 1", weights);
        if (weights == 0 && !kp_valid) return fail(SKMETAL_EINVAL, "no k-means|| distances to sample from");
        if (arena != nullptr) return fail(SKMETAL_EINVAL, "sampling needs the device buffer cache");
        if (n >= (1L << 31)) return fail(SKMETAL_ERANGE, "sampling supports n < 2^31 rows (n=%ld)", n);
        if (ws.p == nullptr) {
            const int nb = ws_blocks(n), nc = ws_chunks(n);
            TRY(grab((void**)&ws.p, size_t(n) * sizeof(double)));
            TRY(grab((void**)&ws.bsum, size_t(nb) * sizeof(float)));
            TRY(grab((void**)&ws.total, sizeof(float)));
            TRY(grab((void**)&ws.ctot, size_t(nc) * sizeof(double)));
            TRY(grab((void**)&ws.cnz, size_t(nc) * sizeof(int)));
            TRY(grab((void**)&ws.pfx, size_t(nc + 1) * sizeof(double)));
            TRY(grab((void**)&ws.nnz, sizeof(long long)));
        }
        ws.n = n;
        ws.w = weights == 0 ? kp_mind : nullptr;
        ws.floor = 1e-30f;
        HIP_TRY(launch_ws_prepare(ws, s), "sampling prepare launch");
        double st[1];
        long long z = 0;
        TRY(download_bytes(*C, ws.pfx + ws_chunks(n), sizeof(double), st, s));
        TRY(download_bytes(*C, ws.nnz, sizeof(long long), &z, s));
        *psum = st[0];
        *nnz = z;
        ws_ready = true;
        return 0;
    }

    // Rows for the m uniforms u after zeroing p at the nz rows `zero`; exact
    // = 1 searches numpy's own cumsum for every draw, exact = 2 gives the
    // certified search a margin of at least 1/(4n) (about half the draws then
    // go to the exact search: both searches in one pass).  *n_exact = draws
    // the certified search left to the exact one.
    int sample_draw(const long* zero, long nz, const double* u, long m, long* out, int exact, int* n_exact)
    {
        if (!ws_ready) return fail(SKMETAL_EINVAL, "sample_draw before sample_prepare");
        if (m < 0 || m > (1L << 24) || nz < 0 || nz > n)
            return fail(SKMETAL_ERANGE, "m=%ld draws or %ld zeroed rows out of range", m, nz);
        if ((m > 0 && (u == nullptr || out == nullptr)) || (nz > 0 && zero == nullptr))
            return fail(SKMETAL_EINVAL, "null pointer argument");
        for (long i = 0; i < m; ++i)
            if (!(u[i] >= 0.0 && u[i] < 1.0)) return fail(SKMETAL_EINVAL, "uniform %ld not in [0, 1)", i);
        for (long i = 0; i < nz; ++i)
            if (zero[i] < 0 || zero[i] >= n) return fail(SKMETAL_EINVAL, "zeroed row %ld not in [0, %ld)", zero[i], n);
        *n_exact = 0;
        if (m == 0) return 0;
        const long need = std::max(m, nz);
        if (need > ws_mcap) {
            const long cap = std::max<long>(need, 2 * ws_mcap);
            for (void* q : {(void*)ws.u, (void*)ws.out, (void*)ws.unsure, (void*)ws.zero}) {
                if (q == nullptr) continue;
                const auto it = std::find(owned.begin(), owned.end(), q);
                if (it != owned.end()) owned.erase(it);
                C->release(q);
            }
            TRY(grab((void**)&ws.u, size_t(cap) * sizeof(double)));
            TRY(grab((void**)&ws.out, size_t(cap) * sizeof(long)));
            TRY(grab((void**)&ws.unsure, size_t(cap) * sizeof(int)));
            TRY(grab((void**)&ws.zero, size_t(cap) * sizeof(long)));
            ws_mcap = cap;
        }
        if (exact < 0 || exact > 2) return fail(SKMETAL_EINVAL, "exact=%d is not 0, 1 or 2", exact);
        ws.m = (int)m;
        ws.nz = (int)nz;
        ws.dmin = exact == 2 ? 0.25 / (double)n : 0.0;
        if (nz > 0) {
            TRY(upload_bytes(*C, zero, size_t(nz) * sizeof(long), const_cast<long*>(ws.zero), s));
            HIP_TRY(launch_ws_zero(ws, s), "sampling zero launch");
        }
        TRY(upload_bytes(*C, u, size_t(m) * sizeof(double), const_cast<double*>(ws.u), s));
        std::vector<int> uns(size_t(m), 1);
        if (exact != 1) {
            HIP_TRY(launch_ws_search(ws, s), "sampling search launch");
            TRY(download_bytes(*C, ws.unsure, size_t(m) * sizeof(int), uns.data(), s));
        }
        long left = 0;
        for (long i = 0; i < m; ++i) left += uns[i] != 0;
        if (left > 0) {
            if (ws.cst == nullptr) {
                TRY(grab((void**)&ws.cst, size_t(ws_chunks(n) + 1) * sizeof(double)));
                TRY(grab((void**)&ws.cseq, size_t(ws_chunks(n)) * sizeof(int)));
            }
            HIP_TRY(launch_ws_exact(ws, exact == 1 ? 1 : 0, s), "sampling exact launch");
        }
        TRY(download_bytes(*C, ws.out, size_t(m) * sizeof(long), out, s));
        *n_exact = (int)left;
        return 0;
    }

    // Full sklearn fit from the current centres: loop, final E-step, inertia.
    int fit(long max_iter, double tol, int flags, int* n_iter_out, double* inertia_out)
    {
        int n_iter = 0, done = 0;
        TRY(run_loop(max_iter, tol, flags, false, &n_iter, &done));
        double in = 0.0;
        if (done != 1)
            TRY(assign_inertia(cen[cur], &in));  // final E-step (_kmeans.py:736-748) and inertia (:749)
        else
            TRY(inertia(&in));
        if (n_iter_out) *n_iter_out = n_iter;
        if (inertia_out) *inertia_out = in;
        return 0;
    }
};

int check_sizes(size_t n, size_t d, size_t k)
{
    if (n == 0 || d == 0 || k == 0) return fail(SKMETAL_EINVAL, "n, d and k must be positive (n=%zu d=%zu k=%zu)", n, d, k);
    if (d > kMaxDim / 4 || k > kMaxDim) return fail(SKMETAL_ERANGE, "d=%zu or k=%zu exceeds the supported range", d, k);
    if (n > (size_t(1) << 40)) return fail(SKMETAL_ERANGE, "n=%zu exceeds the supported range", n);
    return 0;
}

struct Guard {
    std::lock_guard<std::recursive_mutex> lk;
    explicit Guard(Context& c) : lk(c.mu) { g_err.clear(); }
};

// RAII holder for per-call problems built on the shared context.
struct Scoped {
    Lloyd L;
    ~Scoped() { L.destroy(); }
};

}  // namespace

struct skmetal_hip_lloyd {
    Lloyd L;
};

// rocBLAS, opened on the first skmetal_gemm call
namespace {
struct Blas {
    bool tried = false;
    void* so = nullptr;
    rocblas_handle handle = nullptr;
    decltype(&rocblas_create_handle) create = nullptr;
    decltype(&rocblas_set_stream) set_stream = nullptr;
    decltype(&rocblas_sgemm) sgemm = nullptr;
};
Blas g_blas;

int blas_ready(Context& c)
{
    Blas& b = g_blas;
    if (b.handle) return 0;
    if (b.tried) return fail(SKMETAL_ENODEV, "rocBLAS is not available (librocblas could not be opened earlier)");
    b.tried = true;
    for (const char* name : {"librocblas.so.5", "librocblas.so"}) {
        b.so = dlopen(name, RTLD_NOW | RTLD_LOCAL);
        if (b.so) break;
    }
    if (!b.so) return fail(SKMETAL_ENODEV, "skmetal_gemm needs rocBLAS: %s", dlerror());
    b.create = reinterpret_cast<decltype(b.create)>(dlsym(b.so, "rocblas_create_handle"));
    b.set_stream = reinterpret_cast<decltype(b.set_stream)>(dlsym(b.so, "rocblas_set_stream"));
    b.sgemm = reinterpret_cast<decltype(b.sgemm)>(dlsym(b.so, "rocblas_sgemm"));
    if (!b.create || !b.set_stream || !b.sgemm) return fail(SKMETAL_ENODEV, "librocblas lacks rocblas_sgemm");
    rocblas_handle h = nullptr;
    if (b.create(&h) != rocblas_status_success) return fail(SKMETAL_EHIP, "rocblas_create_handle failed");
    if (b.set_stream(h, c.stream) != rocblas_status_success) return fail(SKMETAL_EHIP, "rocblas_set_stream failed");
    b.handle = h;
    return 0;
}
}  // namespace

extern "C" {

const char* skmetal_hip_last_error(void) { return g_err.c_str(); }

int skmetal_init(void)
{
    Context& c = ctx();
    Guard g(c);
    return c.init();
}

int skmetal_warmup(void)
{
    Context& c = ctx();
    Guard g(c);
    TRY(c.init());
    const long n = 300;
    const int d = 6, k = 5;
    std::vector<float> X(static_cast<size_t>(n) * d), C0(static_cast<size_t>(k) * d);
    for (long i = 0; i < n; ++i)
        for (int f = 0; f < d; ++f) X[size_t(i) * d + f] = float((i * 7 + f * 3) % 11) + 0.25f * float(i % k);
    for (int j = 0; j < k; ++j)
        for (int f = 0; f < d; ++f) C0[size_t(j) * d + f] = X[size_t(j * 3) * d + f];
    Scoped sc;
    TRY(sc.L.create(&c, n, d, k));
    TRY(sc.L.load_X(X.data(), true));
    TRY(sc.L.set_centers(C0.data()));
    int it = 0;
    double in = 0.0;
    TRY(sc.L.fit(3, 0.0, kStopStrict, &it, &in));
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return 0;
}

int skmetal_device_info(char* name, int name_capacity, size_t* max_threads, uint8_t* has_unified_memory,
                        uint64_t* recommended_working_set_size)
{
    Context& c = ctx();
    Guard g(c);
    TRY(c.init());
    if (name != nullptr && name_capacity > 0) {
        const size_t m = std::min(c.name.size(), size_t(name_capacity - 1));
        std::memcpy(name, c.name.data(), m);
        name[m] = 0;
    }
    if (max_threads) *max_threads = size_t(c.max_threads);
    if (has_unified_memory) *has_unified_memory = 0;
    if (recommended_working_set_size) *recommended_working_set_size = uint64_t(c.total_mem);
    return 0;
}

int skmetal_hip_release_cache(void)
{
    Context& c = ctx();
    Guard g(c);
    if (c.ready) {
        HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
        c.release_cache();
    }
    return 0;
}

int skmetal_kmeans_assign(const void* X, const void* centroids, void* assignments, size_t n, size_t d, size_t k)
{
    Context& c = ctx();
    Guard g(c);
    if (!X || !centroids || !assignments) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(check_sizes(n, d, k));
    TRY(c.init());
    Scoped sc;
    Lloyd& L = sc.L;
    TRY(L.create(&c, (long)n, (int)d, (int)k));
    TRY(L.load_X(static_cast<const float*>(X), false));
    TRY(L.set_centers(static_cast<const float*>(centroids)));
    TRY(L.assign(L.cen[L.cur], nullptr, nullptr));
    TRY(L.get_labels(static_cast<int32_t*>(assignments)));
    return 0;
}

int skmetal_hip_kmeans_fit(const float* X, float* centroids, int32_t* labels, size_t n, size_t d, size_t k,
                           size_t max_iter, double tol, int flags, int32_t* n_iter_out, double* inertia_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!X || !centroids || !labels) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(check_sizes(n, d, k));
    if (k > n) return fail(SKMETAL_EINVAL, "n_samples=%zu should be >= n_clusters=%zu", n, k);
    if (!(tol >= 0.0)) return fail(SKMETAL_EINVAL, "tol must be >= 0");
    if (max_iter > (size_t(1) << 30)) return fail(SKMETAL_ERANGE, "max_iter too large");
    TRY(c.init());
    Scoped sc;
    Lloyd& L = sc.L;
    TRY(L.create(&c, (long)n, (int)d, (int)k));
    TRY(L.load_X(X, true));
    TRY(L.set_centers(centroids));
    int it = 0;
    double in = 0.0;
    TRY(L.fit((long)max_iter, tol, flags & SKMETAL_FIT_STRICT ? kStopStrict : 0, &it, &in));
    TRY(L.get_labels(labels));
    TRY(L.get_centers(centroids));
    if (n_iter_out) *n_iter_out = it;
    if (inertia_out) *inertia_out = in;
    return 0;
}

// skmetal's own loop contract (KMeansBridge.swift:187-320): up to max_iter
// Lloyd steps; after each, stop when the largest centre shift's fp32 root is
// below tol (:306-310); no label-based stop and no final E-step, so the
// assignments are those of the last step's E-step (against the centres it
// started from) and the centroids those it produced; n_iter = steps run.
// The steps themselves are this library's (X centred on its column mean,
// empty clusters relocated as scikit-learn does, where the reference set
// them to 0).  num_groups sized the reference's partial buffers; unused here.
int skmetal_kmeans_batch_fused(const void* X, void* centroids, void* assignments, size_t n, size_t d, size_t k,
                               size_t num_groups, size_t max_iter, float tol, int32_t* n_iter_out)
{
    (void)num_groups;
    Context& c = ctx();
    Guard g(c);
    if (!X || !centroids || !assignments) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(check_sizes(n, d, k));
    if (k > n) return fail(SKMETAL_EINVAL, "n_samples=%zu should be >= n_clusters=%zu", n, k);
    if (max_iter > (size_t(1) << 30)) return fail(SKMETAL_ERANGE, "max_iter too large");
    TRY(c.init());
    Scoped sc;
    Lloyd& L = sc.L;
    TRY(L.create(&c, (long)n, (int)d, (int)k));
    TRY(L.load_X(static_cast<const float*>(X), true));
    TRY(L.set_centers(static_cast<const float*>(centroids)));
    int it = 0, done = 0;
    TRY(L.run_loop((long)max_iter, (double)tol, kStopMaxShift, false, &it, &done));
    if (max_iter > 0) {
        TRY(L.get_labels(static_cast<int32_t*>(assignments)));
        TRY(L.get_centers(static_cast<float*>(centroids)));
    }
    if (n_iter_out) *n_iter_out = it;
    return 0;
}

int skmetal_hip_kmeans_batch_fused_noalloc(const float* X, float* centroids, int32_t* assignments, size_t n,
                                           size_t d, size_t k, size_t max_iter, float tol, int32_t* n_iter_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!X || !centroids || !assignments) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(check_sizes(n, d, k));
    if (k > n) return fail(SKMETAL_EINVAL, "n_samples=%zu should be >= n_clusters=%zu", n, k);
    if (max_iter > (size_t(1) << 30)) return fail(SKMETAL_ERANGE, "max_iter too large");
    if (!c.ready || c.scratch == nullptr)
        return fail(SKMETAL_EINVAL, "skmetal_init must run first: this entry point does not set the library up");
    if (k > 64) return fail(SKMETAL_ERANGE, "k=%zu: this entry point takes at most 64 clusters", k);
    bool row_ok = false;
    for (const size_t ld : {4, 8, 16, 32, 48, 64, 80, 100}) row_ok = row_ok || d == ld;
    if (!row_ok)
        return fail(SKMETAL_ERANGE, "d=%zu: this entry point takes rows of 4, 8, 16, 32, 48, 64, 80 or 100 floats", d);
    if (fused_ld((int)d, (int)k) != (int)d)
        return fail(SKMETAL_EINVAL,
                    "d=%zu, k=%zu: the fused step kernels are switched off (SKMETAL_HIP_FUSED=0) or could not be "
                    "configured, and this entry point runs only them",
                    d, k);
    if (n > size_t(kNoAllocMaxRows))
        return fail(SKMETAL_ERANGE, "n=%zu: this entry point takes at most %ld rows", n, kNoAllocMaxRows);
    int it = 0;
    if (max_iter > 0) {
        Lloyd L;
        L.arena = static_cast<char*>(c.scratch);
        L.arena_cap = kScratchBytes;
        int rc = L.create_noalloc(&c, (long)n, (int)d, (int)k, X, centroids, assignments);
        int done = 0;
        if (rc == 0) rc = L.run_loop((long)max_iter, (double)tol, kStopMaxShift, false, &it, &done);
        if (rc == 0 && L.cur != 0) {
            const hipError_t e = hipMemcpyAsync(centroids, L.cen[L.cur], k * d * sizeof(float),
                                                hipMemcpyDeviceToDevice, L.s);
            if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(centres)");
        }
        const hipError_t e = hipStreamSynchronize(L.s);
        if (rc == 0 && e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
        if (rc != 0) return rc;
    }
    if (n_iter_out) *n_iter_out = it;
    return 0;
}

static int rowdist_call(const void* X, const void* centroids, const void* assignments, void* dists, size_t n,
                        size_t d, size_t k, double* total)
{
    Context& c = ctx();
    if (!X || !centroids || !assignments) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(check_sizes(n, d, k));
    TRY(c.init());
    // labels are indices into the centroid rows: reject out-of-range values
    const int32_t* lab = static_cast<const int32_t*>(assignments);
    for (size_t i = 0; i < n; ++i)
        if (lab[i] < 0 || size_t(lab[i]) >= k) return fail(SKMETAL_EINVAL, "assignments[%zu]=%d not in [0, %zu)", i, lab[i], k);
    Scoped sc;
    Lloyd& L = sc.L;
    TRY(L.create(&c, (long)n, (int)d, (int)k));
    TRY(L.load_X(static_cast<const float*>(X), false));
    TRY(L.set_centers(static_cast<const float*>(centroids)));
    TRY(upload_bytes(c, assignments, n * sizeof(int32_t), L.labels, L.s));
    if (dists != nullptr) TRY(L.grab((void**)&L.rowout, n * sizeof(float)));
    RowDistArgs r{L.X, L.n, L.ld, L.d, L.cen[L.cur], L.k, L.labels, dists ? L.rowout : nullptr, L.rowpart, L.st};
    HIP_TRY(launch_rowdist(r, L.s), "rowdist launch");
    LoopState hs{};
    TRY(L.read_state(&hs));
    if (total) *total = hs.inertia;
    if (dists != nullptr) TRY(download_bytes(c, L.rowout, n * sizeof(float), dists, L.s));
    return 0;
}

int skmetal_compute_mindists(const void* X, const void* centroids, const void* assignments, void* dists, size_t n,
                             size_t d, size_t k)
{
    Context& c = ctx();
    Guard g(c);
    if (!dists) return fail(SKMETAL_EINVAL, "null pointer argument");
    return rowdist_call(X, centroids, assignments, dists, n, d, k, nullptr);
}

float skmetal_kmeans_inertia(const void* X, const void* centroids, const void* assignments, size_t n, size_t d,
                             size_t k)
{
    Context& c = ctx();
    Guard g(c);
    double total = 0.0;
    if (rowdist_call(X, centroids, assignments, nullptr, n, d, k, &total) != 0) return -1.0f;
    return (float)total;
}

// ---- device-resident handle ----

int skmetal_hip_lloyd_create(size_t n, size_t d, size_t k, skmetal_hip_lloyd** out)
{
    Context& c = ctx();
    Guard g(c);
    if (!out) return fail(SKMETAL_EINVAL, "null pointer argument");
    *out = nullptr;
    TRY(check_sizes(n, d, k));
    if (k > n) return fail(SKMETAL_EINVAL, "n_samples=%zu should be >= n_clusters=%zu", n, k);
    TRY(c.init());
    auto* h = new skmetal_hip_lloyd();
    const int rc = h->L.create(&c, (long)n, (int)d, (int)k);
    if (rc != 0) {
        h->L.destroy();
        delete h;
        return rc;
    }
    *out = h;
    return 0;
}

int skmetal_hip_lloyd_destroy(skmetal_hip_lloyd* h)
{
    if (!h) return 0;
    Context& c = ctx();
    Guard g(c);
    h->L.destroy();
    delete h;
    return 0;
}

int skmetal_hip_lloyd_load(skmetal_hip_lloyd* h, const float* X, int center)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !X) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(h->L.load_X(X, center != 0));
    HIP_TRY(hipStreamSynchronize(h->L.s), "hipStreamSynchronize");
    return 0;
}

int skmetal_hip_lloyd_set_centers(skmetal_hip_lloyd* h, const float* C)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !C) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(h->L.set_centers(C));
    HIP_TRY(hipStreamSynchronize(h->L.s), "hipStreamSynchronize");
    return 0;
}

int skmetal_hip_lloyd_iterate(skmetal_hip_lloyd* h, size_t iters, float* ms_out, float* kernel_ms)
{
    Context& c = ctx();
    Guard g(c);
    if (!h) return fail(SKMETAL_EINVAL, "null pointer argument");
    Lloyd& L = h->L;
    if (kernel_ms) {
        if (iters > kMaxTimedSteps) return fail(SKMETAL_ERANGE, "iterate: kernel timing covers at most 4096 steps");
        // timing-only markers: no system-scope fence (its L2 writeback and
        // invalidation would sit inside the brackets and slow the next kernel);
        // e1, recorded after them and synchronised on, orders them for the host
        while (L.kev.size() < 4 * iters) {
            hipEvent_t e;
            HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreate");
            L.kev.push_back(e);
        }
    }
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreateWithFlags(&e0, hipEventDisableSystemFence), "hipEventCreate");
    HIP_TRY(hipEventCreate(&e1), "hipEventCreate");
    int rc = 0;
    // the loop resets the device state and labels before the timed region
    LoopState hs{};
    rc = L.write_state(hs);
    if (rc == 0) {
        L.kev_base = kernel_ms ? 0 : -1;
        hipError_t er = hipEventRecord(e0, L.s);
        if (er != hipSuccess) rc = hip_fail(er, "hipEventRecord");
        int n_iter = 0, done = 0;
        // e1 is recorded by the loop right after the last step's kernels
        L.batch_end = e1;
        if (rc == 0) rc = L.run_loop((long)iters, 0.0, 0, true, &n_iter, &done);
        L.batch_end = nullptr;
        if (rc == 0 && iters == 0) {
            er = hipEventRecord(e1, L.s);
            if (er != hipSuccess) rc = hip_fail(er, "hipEventRecord");
        }
        L.kev_base = -1;
        hipError_t e = hipEventSynchronize(e1);
        if (rc == 0 && e != hipSuccess) rc = hip_fail(e, "hipEventSynchronize");
        if (rc == 0 && ms_out) {
            e = hipEventElapsedTime(ms_out, e0, e1);
            if (e != hipSuccess) rc = hip_fail(e, "hipEventElapsedTime");
        }
        if (rc == 0 && kernel_ms) {
            // averages over the steps: main kernel, update kernels, finalize
            double sum[3] = {0.0, 0.0, 0.0};
            for (size_t i = 0; i < iters && rc == 0; ++i) {
                for (int j = 0; j < 3; ++j) {
                    float t = 0.f;
                    const hipError_t ee = hipEventElapsedTime(&t, L.kev[4 * i + j], L.kev[4 * i + j + 1]);
                    if (ee != hipSuccess) rc = hip_fail(ee, "hipEventElapsedTime");
                    sum[j] += t;
                }
            }
            for (int j = 0; j < 3; ++j) kernel_ms[j] = iters ? float(sum[j] / double(iters)) : 0.f;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int skmetal_hip_lloyd_run(skmetal_hip_lloyd* h, size_t max_iter, double tol, int flags, int32_t* n_iter_out,
                          double* inertia_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!h) return fail(SKMETAL_EINVAL, "null pointer argument");
    int it = 0;
    double in = 0.0;
    TRY(h->L.fit((long)max_iter, tol, flags & SKMETAL_FIT_STRICT ? kStopStrict : 0, &it, &in));
    if (n_iter_out) *n_iter_out = it;
    if (inertia_out) *inertia_out = in;
    return 0;
}

int skmetal_hip_lloyd_plusplus(skmetal_hip_lloyd* h, size_t n_local_trials, int64_t first_index,
                               const double* uniforms, int64_t* indices_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !indices_out) return fail(SKMETAL_EINVAL, "null pointer argument");
    static_assert(sizeof(long) == sizeof(int64_t), "64-bit long expected");
    TRY(h->L.plusplus((int)std::min<size_t>(n_local_trials, size_t(kPPMaxTrials) + 1), (long)first_index, uniforms,
                      reinterpret_cast<long*>(indices_out)));
    HIP_TRY(hipStreamSynchronize(h->L.s), "hipStreamSynchronize");
    return 0;
}

int skmetal_hip_lloyd_mindists(skmetal_hip_lloyd* h, const int64_t* rows, size_t m, int reset, float* dists_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!h) return fail(SKMETAL_EINVAL, "null pointer argument");
    if (m > (size_t(1) << 30)) return fail(SKMETAL_ERANGE, "m=%zu candidate rows out of range", m);
    TRY(h->L.mindists(reinterpret_cast<const long*>(rows), (long)m, reset, dists_out));
    HIP_TRY(hipStreamSynchronize(h->L.s), "hipStreamSynchronize");
    return 0;
}

int skmetal_hip_lloyd_sample_prepare(skmetal_hip_lloyd* h, int weights, double* p_sum_out, int64_t* nonzero_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !p_sum_out || !nonzero_out) return fail(SKMETAL_EINVAL, "null pointer argument");
    long long z = 0;
    TRY(h->L.sample_prepare(weights, p_sum_out, &z));
    *nonzero_out = (int64_t)z;
    return 0;
}

int skmetal_hip_lloyd_sample_draw(skmetal_hip_lloyd* h, const int64_t* zero_rows, size_t n_zero, const double* uniforms,
                                  size_t m, int64_t* rows_out, int exact, int* n_exact_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!h) return fail(SKMETAL_EINVAL, "null pointer argument");
    if (m > (size_t(1) << 24) || n_zero > (size_t(1) << 40))
        return fail(SKMETAL_ERANGE, "m=%zu draws or %zu zeroed rows out of range", m, n_zero);
    int ne = 0;
    TRY(h->L.sample_draw(reinterpret_cast<const long*>(zero_rows), (long)n_zero, uniforms, (long)m,
                         reinterpret_cast<long*>(rows_out), exact, &ne));
    HIP_TRY(hipStreamSynchronize(h->L.s), "hipStreamSynchronize");
    if (n_exact_out) *n_exact_out = ne;
    return 0;
}

int skmetal_hip_kmeans_plusplus(const float* X, size_t n, size_t d, size_t k, size_t n_local_trials,
                                int64_t first_index, const double* uniforms, int64_t* indices_out)
{
    Context& c = ctx();
    Guard g(c);
    if (!X || !indices_out) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(check_sizes(n, d, k));
    if (k > n) return fail(SKMETAL_EINVAL, "n_samples=%zu should be >= n_clusters=%zu", n, k);
    TRY(c.init());
    Scoped sc;
    Lloyd& L = sc.L;
    TRY(L.create(&c, (long)n, (int)d, (int)k));
    TRY(L.load_X(X, false));
    TRY(L.plusplus((int)std::min<size_t>(n_local_trials, size_t(kPPMaxTrials) + 1), (long)first_index, uniforms,
                   reinterpret_cast<long*>(indices_out)));
    return 0;
}

int skmetal_hip_kmeans_transform(const float* X, const float* centroids, float* out, size_t n, size_t d, size_t k)
{
    Context& c = ctx();
    Guard g(c);
    if (!X || !centroids || !out) return fail(SKMETAL_EINVAL, "null pointer argument");
    TRY(check_sizes(n, d, k));
    TRY(c.init());
    const int ld = ((int)d + 3) & ~3;
    // rows per pass: the pass's X rows and distances stay under ~512 MB
    const size_t row_bytes = size_t(ld + k) * sizeof(float);
    long rows = (long)std::max<size_t>(64, (size_t(512) << 20) / row_bytes) & ~63L;
    rows = std::min<long>(rows, ((long)n + 63) & ~63L);
    struct Bufs {
        Context& c;
        std::vector<void*> p;
        ~Bufs() { for (void* q : p) c.release(q); }
        int get(void** out, size_t bytes)
        {
            TRY(c.alloc(out, bytes));
            p.push_back(*out);
            return 0;
        }
    } b{c, {}};
    float *dX = nullptr, *dC = nullptr, *dO = nullptr;
    double* dcc = nullptr;
    TRY(b.get((void**)&dX, size_t(rows) * ld * sizeof(float)));
    TRY(b.get((void**)&dC, k * size_t(ld) * sizeof(float)));
    TRY(b.get((void**)&dcc, k * sizeof(double)));
    TRY(b.get((void**)&dO, size_t(rows) * k * sizeof(float)));
    double* dfrag = nullptr;
    if (transform_mm_path(ld)) TRY(b.get((void**)&dfrag, (k + 15) / 16 * 16 * size_t(ld) * sizeof(double)));
    TRY(upload_rows(c, centroids, (long)k, (int)d, ld, dC, c.stream));
    for (long r = 0; r < (long)n; r += rows) {
        const long m = std::min<long>(rows, (long)n - r);
        TRY(upload_rows(c, X + size_t(r) * d, m, (int)d, ld, dX, c.stream));
        TransformArgs a{dX, m, ld, dC, (int)k, dcc, dO, dfrag, c.num_cu};
        HIP_TRY(launch_transform(a, c.stream), "transform launch");
        TRY(download_bytes(c, dO, size_t(m) * k * sizeof(float), out + size_t(r) * k, c.stream));
    }
    return 0;
}

// ---------------------------------------------------------------------------
// skmetal_gemm: the reference's fp32 GEMM entry point (its MPS matrix
// multiply), which skmetal's MetalKMeans.transform calls for x.c^T.  A plain
// library GEMM: rocBLAS sgemm on the library's stream, with librocblas opened
// on the first call (the rest of the library does not depend on it).
// ---------------------------------------------------------------------------

int skmetal_gemm(const void* A, const void* B, void* C, size_t M, size_t N, size_t K, float alpha, float beta,
                 int transpose_A, int transpose_B)
{
    Context& c = ctx();
    Guard g(c);
    if (!A || !B || !C) return fail(SKMETAL_EINVAL, "null pointer argument");
    if (M == 0 || N == 0 || K == 0) return fail(SKMETAL_EINVAL, "M, N and K must be positive (M=%zu N=%zu K=%zu)", M, N, K);
    const size_t lim = size_t(INT32_MAX);
    if (M > lim || N > lim || K > lim || M * K > (size_t(1) << 36) || K * N > (size_t(1) << 36) ||
        M * N > (size_t(1) << 36))
        return fail(SKMETAL_ERANGE, "gemm sizes too large (M=%zu N=%zu K=%zu)", M, N, K);
    TRY(c.init());
    TRY(blas_ready(c));
    struct Bufs {
        Context& c;
        std::vector<void*> p;
        ~Bufs() { for (void* q : p) c.release(q); }
        int get(void** out, size_t bytes)
        {
            TRY(c.alloc(out, bytes));
            p.push_back(*out);
            return 0;
        }
    } b{c, {}};
    float *dA = nullptr, *dB = nullptr, *dC = nullptr;
    TRY(b.get((void**)&dA, M * K * sizeof(float)));
    TRY(b.get((void**)&dB, K * N * sizeof(float)));
    TRY(b.get((void**)&dC, M * N * sizeof(float)));
    TRY(upload_bytes(c, A, M * K * sizeof(float), dA, c.stream));
    TRY(upload_bytes(c, B, K * N * sizeof(float), dB, c.stream));
    // beta == 0 ignores C's contents (the caller's C may be uninitialised)
    if (beta != 0.f) TRY(upload_bytes(c, C, M * N * sizeof(float), dC, c.stream));
    // row-major C = op(A) op(B) is column-major C^T = op(B)^T op(A)^T: the
    // row-major buffers read as column-major are the transposes
    const rocblas_operation ta = transpose_A ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation tb = transpose_B ? rocblas_operation_transpose : rocblas_operation_none;
    const int lda = (int)(transpose_A ? M : K), ldb = (int)(transpose_B ? K : N);
    if (g_blas.sgemm(g_blas.handle, tb, ta, (int)N, (int)M, (int)K, &alpha, dB, ldb, dA, lda, &beta, dC, (int)N) !=
        rocblas_status_success)
        return fail(SKMETAL_EHIP, "rocblas_sgemm failed");
    return download_bytes(c, dC, M * N * sizeof(float), C, c.stream);
}

// ---------------------------------------------------------------------------
// The other names of skmetal's ctypes registry (skmetal/_bridge.py:107-345):
// its loader binds every one of them when the library loads, so they are
// exported; each returns SKMETAL_ENOSYS (skmetal's wrappers then raise
// RuntimeError("<name> failed with code 7"), as for any failed call).
// ---------------------------------------------------------------------------
#define SKM_NOT_PROVIDED(name) return fail(SKMETAL_ENOSYS, "%s is not provided: libskmetal_hip.so is skmetal's KMeans path", name)

int skmetal_pairwise_distance(const void*, void*, size_t, size_t) { SKM_NOT_PROVIDED("skmetal_pairwise_distance"); }
int skmetal_scaler_fit(const void*, void*, void*, size_t, size_t) { SKM_NOT_PROVIDED("skmetal_scaler_fit"); }
int skmetal_column_minmax(const void*, void*, void*, size_t, size_t) { SKM_NOT_PROVIDED("skmetal_column_minmax"); }
int skmetal_fista_fit(const void*, const void*, void*, size_t, size_t, float, float, float, int32_t, int32_t*)
{
    SKM_NOT_PROVIDED("skmetal_fista_fit");
}
int skmetal_column_transform(const void*, void*, const void*, const void*, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_column_transform");
}
int skmetal_sv_init(void*, size_t) { SKM_NOT_PROVIDED("skmetal_sv_init"); }
int skmetal_sv_hook(void*, const void*, size_t, size_t) { SKM_NOT_PROVIDED("skmetal_sv_hook"); }
int skmetal_sv_shortcut(void*, size_t) { SKM_NOT_PROVIDED("skmetal_sv_shortcut"); }
int skmetal_knn_vote_classify(const void*, const void*, void*, size_t, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_knn_vote_classify");
}
int skmetal_knn_vote_regress(const void*, const void*, void*, size_t, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_knn_vote_regress");
}
int skmetal_knn_vote_classify_weighted(const void*, const void*, const void*, void*, size_t, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_knn_vote_classify_weighted");
}
int skmetal_knn_vote_regress_weighted(const void*, const void*, const void*, void*, size_t, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_knn_vote_regress_weighted");
}
int skmetal_knn_tiled_kneighbors(const void*, const void*, void*, void*, size_t, size_t, size_t, size_t, size_t,
                                 int32_t)
{
    SKM_NOT_PROVIDED("skmetal_knn_tiled_kneighbors");
}
int skmetal_rbf_kernel_square(const void*, void*, float, size_t, size_t) { SKM_NOT_PROVIDED("skmetal_rbf_kernel_square"); }
int skmetal_rbf_kernel_cross(const void*, const void*, void*, float, size_t, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_rbf_kernel_cross");
}
int skmetal_tree_predict_all(const void*, const void*, const void*, const void*, const void*, const void*, const void*,
                             const void*, const void*, const void*, void*, size_t, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_tree_predict_all");
}
int skmetal_svc_predict_binary(const void*, const void*, const void*, const void*, void*, size_t, size_t, size_t, float)
{
    SKM_NOT_PROVIDED("skmetal_svc_predict_binary");
}
int skmetal_logreg_irls_fit(const void*, const void*, void*, float, float, int32_t, int32_t, size_t, size_t, int32_t*)
{
    SKM_NOT_PROVIDED("skmetal_logreg_irls_fit");
}
int skmetal_logreg_lbfgs_fit(const void*, const void*, void*, float, float, int32_t, int32_t, size_t, size_t, int32_t*)
{
    SKM_NOT_PROVIDED("skmetal_logreg_lbfgs_fit");
}
int skmetal_ridge_fit_solve(const void*, const void*, void*, void*, float, size_t, size_t)
{
    SKM_NOT_PROVIDED("skmetal_ridge_fit_solve");
}
int skmetal_multinomial_lbfgs_fit(const void*, const void*, void*, float, float, int32_t, size_t, size_t, size_t,
                                  int32_t*)
{
    SKM_NOT_PROVIDED("skmetal_multinomial_lbfgs_fit");
}
int skmetal_minmax_transform(const void*, void*, const void*, const void*, size_t, size_t, float, float)
{
    SKM_NOT_PROVIDED("skmetal_minmax_transform");
}
int skmetal_convert_f32_to_f16(const void*, void*, size_t) { SKM_NOT_PROVIDED("skmetal_convert_f32_to_f16"); }
int skmetal_convert_f16_to_f32(const void*, void*, size_t) { SKM_NOT_PROVIDED("skmetal_convert_f16_to_f32"); }
int skmetal_gemm_f16(const void*, const void*, void*, size_t, size_t, size_t) { SKM_NOT_PROVIDED("skmetal_gemm_f16"); }
#undef SKM_NOT_PROVIDED

int skmetal_hip_column_variance(const float* X, size_t n, size_t d, float* out)
{
    if (!X || !out) return fail(SKMETAL_EINVAL, "null pointer argument");
    if (n == 0 || d == 0) return fail(SKMETAL_EINVAL, "n and d must be positive (n=%zu d=%zu)", n, d);
    if (d > (size_t(1) << 30) || n > (size_t(1) << 40)) return fail(SKMETAL_ERANGE, "n=%zu or d=%zu too large", n, d);
    column_variance_f32(X, (long)n, (int)d, out);
    return 0;
}

int skmetal_hip_lloyd_max_abs(skmetal_hip_lloyd* h, float* out)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !out) return fail(SKMETAL_EINVAL, "null pointer argument");
    if (!h->L.xmax_known) TRY(h->L.measure_xmax());
    *out = h->L.xmax;
    return 0;
}

int skmetal_hip_lloyd_info(skmetal_hip_lloyd* h, int* fused, int* partials)
{
    if (!h) return fail(SKMETAL_EINVAL, "null pointer argument");
    const Lloyd& L = h->L;
    if (fused) *fused = (L.fblocks > 0 ? (L.split_on && L.f3cap ? 2 : 1) : 0) | (L.split_on && L.a3cap ? 4 : 0);
    if (partials) *partials = h->L.fblocks > 0 ? h->L.fblocks : h->L.sg.on ? (int)h->L.sg.nchunks : h->L.ug.R;
    return 0;
}

int skmetal_hip_lloyd_get_centers(skmetal_hip_lloyd* h, float* C)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !C) return fail(SKMETAL_EINVAL, "null pointer argument");
    return h->L.get_centers(C);
}

int skmetal_hip_lloyd_get_labels(skmetal_hip_lloyd* h, int32_t* labels)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !labels) return fail(SKMETAL_EINVAL, "null pointer argument");
    return h->L.get_labels(labels);
}

int skmetal_hip_lloyd_inertia(skmetal_hip_lloyd* h, double* out)
{
    Context& c = ctx();
    Guard g(c);
    if (!h || !out) return fail(SKMETAL_EINVAL, "null pointer argument");
    return h->L.inertia(out);
}

}  // extern "C"
