// inv_hip.hip -- host side of libinvision_hip.so (the C ABI in include/inv_hip.h).
//
// One library stream (default priority), one mutex: calls are synchronous on
// return unless INV_FLAG_ASYNC, and concurrent calls are serialized, matching
// the reference's single-threaded callers (src/quicknn_transformers.pas:1205,
// 1304).  The library owns all device memory it uses: weights uploaded once
// into handles, plus grow-only workspaces for staged activations, outputs,
// split-K partials and counters.  Host buffers move through two pinned bounce
// buffers, so read-only mmap pointers (src/safetensor.pas:308-317) need no
// registration.
#include "../../include/inv_hip.h"

#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdlib.h>
#include <sys/stat.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "attention.hpp"
#include "convert_kernels.hpp"
#include "host_convert.hpp"
#include "gemm_configs.hpp"
#include "gemm_kernel.hpp"

namespace {

thread_local std::string t_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

}  // namespace

// Error reporting for the library's other translation units (safetensors.cpp):
// records the message for inv_hip_last_error on this thread.  Not exported.
extern "C" __attribute__((visibility("hidden"))) int inv_hip_internal_fail(int code, const char *msg) {
    return fail(code, "%s", msg);
}

namespace {

#define HIPCHK(expr)                                                                         \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess) return fail(INV_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define TRY(expr)              \
    do {                       \
        int rc_ = (expr);      \
        if (rc_) return rc_;   \
    } while (0)

constexpr uint32_t kWeightMagic = 0x57484950u;  // "WHIP"
constexpr size_t kPinChunk = 32u << 20;

// Host-side copies into and out of the pinned bounce buffers, spread over a
// few threads: one thread's memcpy moves ~14 GB/s, well below what PCIe moves,
// and with host fp32 activations (the reference's calling convention) these
// copies are the whole cost of a call.  The calling thread takes slices too.
class CopyPool {
public:
    ~CopyPool() { stop_all(); }
    void start(int nthreads) {
        for (int i = 0; i + 1 < nthreads; ++i) workers_.emplace_back([this] { loop(); });
    }
    void stop_all() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
        workers_.clear();
        stop_ = false;
    }
    int threads() const { return (int)workers_.size() + 1; }
    // fn(i) for every i in [0, count); returns when all are done and no worker
    // holds fn any more.
    void parallel_for(int count, const std::function<void(int)> &fn) {
        if (workers_.empty() || count <= 1) {
            for (int i = 0; i < count; ++i) fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            job_ = &fn;
            total_ = count;
            next_.store(0);
            active_ = (int)workers_.size();
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return active_ == 0; });
        job_ = nullptr;
    }

private:
    void work() {
        for (int i; (i = next_.fetch_add(1)) < total_;) (*job_)(i);
    }
    void loop() {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            lk.unlock();
            work();
            lk.lock();
            if (--active_ == 0) done_.notify_one();
        }
    }
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    const std::function<void(int)> *job_ = nullptr;
    std::atomic<int> next_{0};
    int total_ = 0, active_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};

CopyPool g_copy;

// memcpy of n bytes (or of `rows` rows of `width` bytes between pitches) on the pool.
void par_copy_rows(char *dst, size_t dpitch, const char *src, size_t spitch, int64_t rows, size_t width) {
    const size_t total = (size_t)rows * width;
    const int parts = (int)std::min<size_t>((size_t)g_copy.threads() * 2, std::max<size_t>(1, total >> 20));
    if (dpitch == width && spitch == width) {
        const size_t per = (total / parts + 63) & ~(size_t)63;
        g_copy.parallel_for(parts, [&](int i) {
            const size_t off = (size_t)i * per;
            if (off < total) memcpy(dst + off, src + off, std::min(per, total - off));
        });
    } else {
        const int64_t per = (rows + parts - 1) / parts;
        g_copy.parallel_for(parts, [&](int i) {
            for (int64_t r = (int64_t)i * per; r < std::min<int64_t>(rows, (int64_t)(i + 1) * per); ++r)
                memcpy(dst + r * dpitch, src + r * spitch, width);
        });
    }
}

// Host fp32 rows rounded to bf16 rows (nearest even, the device's rounding)
// on the pool: dst [rows x ldd], columns cols..cols_pad-1 zero.  Rounding while
// copying into the bounce buffers halves the bytes that cross PCIe.
void par_cvt_rows(uint16_t *dst, int64_t ldd, const float *src, int64_t lds, int64_t rows, int64_t cols,
                  int64_t cols_pad) {
    const size_t total = (size_t)rows * (size_t)cols * 4;
    const int parts = (int)std::min<size_t>((size_t)g_copy.threads() * 2, std::max<size_t>(1, total >> 20));
    if (rows >= parts) {
        const int64_t per = (rows + parts - 1) / parts;
        g_copy.parallel_for(parts, [&](int i) {
            const int64_t r0 = (int64_t)i * per, nr = std::min<int64_t>(per, rows - r0);
            if (nr > 0) inv::host_f32_to_bf16_rows(dst + r0 * ldd, ldd, src + r0 * lds, lds, nr, cols, cols_pad);
        });
    } else {  // few wide rows: column slices of every row (multiples of 16 columns)
        const int64_t per = ((cols_pad + parts - 1) / parts + 15) / 16 * 16;
        g_copy.parallel_for(parts, [&](int i) {
            const int64_t c0 = (int64_t)i * per;
            if (c0 >= cols_pad) return;
            const int64_t cp = std::min<int64_t>(per, cols_pad - c0);
            const int64_t cc = std::max<int64_t>(0, std::min<int64_t>(cp, cols - c0));
            inv::host_f32_to_bf16_rows(dst + c0, ldd, src + std::min(c0, cols), lds, rows, cc, cp);
        });
    }
}

struct Buf {
    void *p = nullptr;
    size_t cap = 0;
};

struct State {
    bool init = false;
    int device = -1;
    hipStream_t stream = nullptr;
    hipEvent_t tim0 = nullptr, tim1 = nullptr, st0 = nullptr, st1 = nullptr;
    hipEvent_t pin_ev[2] = {nullptr, nullptr};
    void *pin[2] = {nullptr, nullptr};
    // Row-band pipeline of a host-pointer projection, made on its first use:
    // an upload and a download stream (default priority), their events, and two
    // pinned bounce buffers for the output (the input uses pin[]).
    struct {
        bool tried = false, ready = false;
        hipStream_t up = nullptr, down = nullptr;
        hipEvent_t start = nullptr, in_ev[2] = {nullptr, nullptr}, gemm_ev[2] = {nullptr, nullptr},
                   out_ev[2] = {nullptr, nullptr};
        void *pin_out[2] = {nullptr, nullptr};
    } pipe;
    int cu_count = 0, clock_khz = 0;
    char name[256] = {0};
    Buf xin, x16, w16, win, yout, cin, bias, gate;
    Buf aq, ak, avt, aqin, akin, avin;  // attention operands (bf16) and their staging
    Buf nvec;                           // normalisation scale/shift vectors from host
    Buf amask;                          // attention key mask from host
    Buf hx, hvec;                       // head norm / rotary: X and the weight + tables from host
    Buf csrc, ccol, cdst;               // convolution: images from host, patch matrix, output for host
    Buf cimg, cfilt;                    // implicit convolution: NHWC bf16 image, tap-major filter
    // Split/stream-K partial sums and arrival counters: uncached device memory
    // (coherent across XCDs without L2 maintenance).  Such memory is never
    // freed once a kernel has read it: outgrown buffers are retired, not freed.
    Buf partial, counters;
    std::vector<void *> retired_uncached;
    int sgemm_prec = INV_PREC_SPLIT_AB;
    bool stats = false;
    int64_t calls = 0;
    double gemm_ms = 0.0, flops = 0.0;
    std::vector<inv_weight_s *> weights;
    unsigned char *scratch = nullptr;  // device address of `scratch` on g.device
    // Device memory the library holds (workspaces, weights, inv_hip_malloc
    // buffers), and an optional cap on it (INV_HIP_ALLOC_LIMIT_MB at
    // inv_hip_init; 0: none): an allocation past the cap fails with
    // INV_ERR_OOM as a failed hipMalloc would.
    std::unordered_map<void *, size_t> allocs;
    size_t alloc_bytes = 0, alloc_cap = 0;
    size_t alloc_base = 0;  // bytes held when inv_hip_init ran (the cap counts from there)
    // The device weight cache: one entry per (file identity, tensor, bias, flags).
    struct CacheEntry {
        std::string key;
        inv_weight_s *w;
        uint64_t last_use;
        size_t bytes;
    };
    std::vector<CacheEntry> cache;
    size_t cache_bytes = 0;
    int64_t cache_budget = 0;  // bytes; 0: unlimited
    uint64_t cache_clock = 0;
    int64_t cache_hits = 0, cache_misses = 0, cache_uploaded = 0;
};

State g;
std::mutex g_mu;

// The no-allocation entry point's scratch: one array per GPU the library runs
// on, held until the process ends.  Host code never uses its name as an
// address (in host code it is a stand-in symbol): g.scratch holds the device
// address from hipGetSymbolAddress, looked up at inv_hip_init.
//   [0, kScratchCounters)                split-K arrival counters (u32)
//   [kScratchCounters, +kScratchBias)     a bias staged to 16-byte alignment
//   [kScratchCounters + kScratchBias, end)  staged activations, then split-K partial sums
constexpr size_t kScratchCounters = 64u << 10;
constexpr size_t kScratchBias = 256u << 10;
static __device__ __align__(256) unsigned char scratch[INV_NOALLOC_SCRATCH_BYTES];

__global__ void fill_zero_u32(unsigned *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace

struct inv_weight_s {
    uint32_t magic;
    uint16_t *w;   // [rows x ldw] bf16, zero padded beyond K
    float *bias;   // [rows] or null
    int64_t N, K, ldw;
    int gated;     // gate/up pair for INV_EPI_SWIGLU: rows = 2 * N rounded up to 128 per half,
                   // interleaved in 128-row blocks (gate block b at rows 256b, its up block at 256b + 128)
    int64_t rows;  // device rows (N unless gated)
    // Weight cache (inv_hip_weight_cache_get): a cached handle belongs to the
    // cache; inv_hip_weight_free releases one reference instead of freeing.
    bool cached = false;
    bool detached = false;  // dropped from the cache while referenced: freed on its last release
    int refs = 0;           // outstanding references from inv_hip_weight_cache_get
};

namespace {

inline int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Every device allocation of the library goes through dev_alloc / dev_free
// (the cap and the byte count).  uncached: hipDeviceMallocUncached memory.
int dev_alloc(void **p, size_t bytes, const char *what, bool uncached = false) {
    *p = nullptr;
    if (g.alloc_cap && g.alloc_bytes - g.alloc_base + bytes > g.alloc_cap)
        return fail(INV_ERR_OOM, "%s: %zu bytes would exceed the allocation cap (INV_HIP_ALLOC_LIMIT_MB: %zu of "
                    "%zu bytes in use)", what, bytes, g.alloc_bytes - g.alloc_base, g.alloc_cap);
    const hipError_t e = uncached ? hipExtMallocWithFlags(p, bytes, hipDeviceMallocUncached) : hipMalloc(p, bytes);
    if (e != hipSuccess || !*p) {
        (void)hipGetLastError();
        *p = nullptr;
        return fail(INV_ERR_OOM, "%s: device allocation of %zu bytes failed", what, bytes);
    }
    g.allocs[*p] = bytes;
    g.alloc_bytes += bytes;
    return INV_OK;
}

void dev_free(void *p) {
    if (!p) return;
    auto it = g.allocs.find(p);
    if (it != g.allocs.end()) {
        g.alloc_bytes -= it->second;
        g.allocs.erase(it);
    }
    (void)hipFree(p);
}

int ensure(Buf &b, size_t bytes) {
    if (b.cap >= bytes) return INV_OK;
    if (b.p) {
        HIPCHK(hipStreamSynchronize(g.stream));
        dev_free(b.p);
        b.p = nullptr;
        b.cap = 0;
    }
    size_t nb = (size_t)round_up((int64_t)std::max<size_t>(bytes, 1), 2 << 20);
    TRY(dev_alloc(&b.p, nb, "workspace"));
    b.cap = nb;
    return INV_OK;
}

// Grow-only uncached buffer; the old one is retired (kept until process exit).
int ensure_uncached(Buf &b, size_t bytes, bool zero) {
    if (b.cap >= bytes) return INV_OK;
    size_t nb = (size_t)round_up((int64_t)std::max<size_t>(bytes, 1), 2 << 20);
    void *p = nullptr;
    TRY(dev_alloc(&p, nb, "split-K workspace", true));
    if (zero) HIPCHK(hipMemsetAsync(p, 0, nb, g.stream));
    if (b.p) g.retired_uncached.push_back(b.p);
    b.p = p;
    b.cap = nb;
    return INV_OK;
}

void release(Buf &b) {
    dev_free(b.p);
    b.p = nullptr;
    b.cap = 0;
}

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

// The serial copies through the bounce buffers go in pieces of about this
// many bytes (whole rows, at most a bounce buffer), two in flight: the host
// side of one piece (a copy or a rounding into pinned memory) runs while the
// DMA moves its neighbour, so pieces much smaller than a buffer leave less of
// either exposed at the ends.  INV_HIP_COPY_CHUNK_MB changes it (1-32).
size_t copy_chunk() {
    const int mb = env_int("INV_HIP_COPY_CHUNK_MB", 8);
    return (size_t)std::max(1, std::min(32, mb)) << 20;
}

// Host rows -> contiguous device rows, through the pinned bounce buffers.
// rows x width bytes; host rows are `pitch` bytes apart.
int h2d_rows(void *dev, const void *host, int64_t rows, size_t width, size_t pitch) {
    const char *src = (const char *)host;
    char *dst = (char *)dev;
    int k = 0;
    if (width > kPinChunk) {  // very wide rows: one row at a time, in pieces
        for (int64_t r = 0; r < rows; ++r)
            for (size_t off = 0; off < width; off += kPinChunk) {
                size_t n = std::min(kPinChunk, width - off);
                HIPCHK(hipEventSynchronize(g.pin_ev[k]));
                par_copy_rows((char *)g.pin[k], n, src + r * pitch + off, n, 1, n);
                HIPCHK(hipMemcpyAsync(dst + r * width + off, g.pin[k], n, hipMemcpyHostToDevice, g.stream));
                HIPCHK(hipEventRecord(g.pin_ev[k], g.stream));
                k ^= 1;
            }
        return INV_OK;
    }
    const int64_t rows_per = std::max<int64_t>(1, (int64_t)(copy_chunk() / width));
    for (int64_t r0 = 0; r0 < rows; r0 += rows_per) {
        const int64_t nr = std::min(rows_per, rows - r0);
        HIPCHK(hipEventSynchronize(g.pin_ev[k]));
        char *pb = (char *)g.pin[k];
        par_copy_rows(pb, width, src + r0 * pitch, pitch, nr, width);
        HIPCHK(hipMemcpyAsync(dst + r0 * width, pb, (size_t)nr * width, hipMemcpyHostToDevice, g.stream));
        HIPCHK(hipEventRecord(g.pin_ev[k], g.stream));
        k ^= 1;
    }
    return INV_OK;
}

// Host fp32 rows (ld floats apart) -> contiguous device bf16 rows of cols_pad
// (zero padded), rounded by the host while they are copied into the bounce
// buffers.  Rows of up to one bounce buffer (cols_pad * 2 <= kPinChunk).
int h2d_rows_bf16(uint16_t *dev, const float *host, int64_t rows, int64_t cols, int64_t ld, int64_t cols_pad) {
    const size_t width = (size_t)cols_pad * 2;
    if (width > kPinChunk) return fail(INV_ERR_ARG, "internal: bf16 row of %zu bytes above a bounce buffer", width);
    const int64_t rows_per = std::max<int64_t>(1, (int64_t)(copy_chunk() / width));
    int k = 0;
    for (int64_t r0 = 0; r0 < rows; r0 += rows_per) {
        const int64_t nr = std::min(rows_per, rows - r0);
        HIPCHK(hipEventSynchronize(g.pin_ev[k]));
        par_cvt_rows((uint16_t *)g.pin[k], cols_pad, host + r0 * ld, ld, nr, cols, cols_pad);
        HIPCHK(hipMemcpyAsync(dev + r0 * cols_pad, g.pin[k], (size_t)nr * width, hipMemcpyHostToDevice, g.stream));
        HIPCHK(hipEventRecord(g.pin_ev[k], g.stream));
        k ^= 1;
    }
    return INV_OK;
}

// Contiguous device rows -> host rows `pitch` bytes apart (the bytes between
// rows are not touched).  Synchronous.
int d2h_rows(void *host, const void *dev, int64_t rows, size_t width, size_t pitch) {
    char *dst = (char *)host;
    const char *src = (const char *)dev;
    struct Piece {
        int64_t r0, nr;
        size_t off, n;
    };
    std::vector<Piece> pieces;
    if (width > kPinChunk) {
        for (int64_t r = 0; r < rows; ++r)
            for (size_t off = 0; off < width; off += kPinChunk) pieces.push_back({r, 1, off, std::min(kPinChunk, width - off)});
    } else {
        const int64_t rows_per = std::max<int64_t>(1, (int64_t)(copy_chunk() / width));
        for (int64_t r0 = 0; r0 < rows; r0 += rows_per) {
            int64_t nr = std::min(rows_per, rows - r0);
            pieces.push_back({r0, nr, 0, (size_t)nr * width});
        }
    }
    auto drain = [&](size_t i) -> int {
        const Piece &pc = pieces[i];
        HIPCHK(hipEventSynchronize(g.pin_ev[i & 1]));
        const char *pb = (const char *)g.pin[i & 1];
        if (pc.nr == 1 && width > kPinChunk) {
            par_copy_rows(dst + pc.r0 * pitch + pc.off, pc.n, pb, pc.n, 1, pc.n);
        } else {
            par_copy_rows(dst + pc.r0 * pitch, pitch, pb, width, pc.nr, width);
        }
        return INV_OK;
    };
    for (size_t i = 0; i < pieces.size(); ++i) {
        const Piece &pc = pieces[i];
        const char *s = (width > kPinChunk) ? src + pc.r0 * width + pc.off : src + pc.r0 * width;
        HIPCHK(hipMemcpyAsync(g.pin[i & 1], s, pc.n, hipMemcpyDeviceToHost, g.stream));
        HIPCHK(hipEventRecord(g.pin_ev[i & 1], g.stream));
        if (i >= 1) TRY(drain(i - 1));
    }
    if (!pieces.empty()) TRY(drain(pieces.size() - 1));
    return INV_OK;
}

// ---------------------------------------------------------------------------
// GEMM launch
// ---------------------------------------------------------------------------

struct TileChoice {
    int cfg;    // index into the instantiated tile configurations
    int mode;   // inv::GRID_TILES, GRID_SPLITK or GRID_STREAMK
    int count;  // split-K: splits per tile; stream-K: persistent workgroups
};

// Instantiated tile configurations (gemm_configs.hpp).
struct CfgMeta {
    int tn, tm, threads, acc_regs, bk, lds;
    bool reg_staged;  // RsCfg: register-staged main loop
    bool swiglu_ok;   // 256-row tiles over two wave columns with a staged epilogue
    bool staged_epi;  // epilogue through LDS (the one that adds a per-row bias)
    hipError_t (*launch)(const inv::GemmParams &, int, int, int, hipStream_t);
};
#define INV_META(id)                                                                        \
    {INV_CFG_##id::TN,       INV_CFG_##id::TM,  INV_CFG_##id::NTHREADS, INV_CFG_##id::ACC_REGS, \
     INV_CFG_##id::BK,       INV_CFG_##id::LDS_BYTES, INV_CFG_##id::REG_STAGED, INV_CFG_##id::SWIGLU_OK,      \
     INV_CFG_##id::STAGED_EPI, &inv_gemm_launch_##id},
const CfgMeta kCfg[INV_GEMM_NUM_CONFIGS] = {INV_GEMM_CONFIG_IDS(INV_META)};
#undef INV_META
constexpr int kNumCfg = INV_GEMM_NUM_CONFIGS;

// Workgroups of configuration m resident per CU (LDS is the binding limit).
int cfg_occupancy(const CfgMeta &m) { return std::max(1, std::min(2, (160 * 1024) / m.lds)); }

// Pick a tile shape and how the grid covers it (rules from measurements on
// MI355X, 256 CUs):
//  - at least 3/4 of a round of 256x256 tiles: the 256x256 tile of 8 waves on
//    16x16 MFMAs, two waves per SIMD (configuration 17), or the 256x224 one of 4
//    waves (configuration 16), by last-round fill and edge padding, 17 doing
//    ~10% more per tile.  Sustained, in one run (TFLOP/s, 16 / 17, and the
//    32x32-MFMA 256x256 tile, configuration 8, that 17 replaced):
//    9216x3840x15360 1157 / 1208 (8: 1158), 9216x3840x11520 1150 / 1217 (1168),
//    2048x3840x15360 1021 / 1241 (1192), 9216x15360x3840 1122 / 1088 (1047),
//    9216x3840x3840 1125 / 1054 (993), c2 1188 / 1180 (1124: 756 tiles = 2.95
//    rounds against 648 = 2.53);
//  - M <= 128 and half a round of 256x128 tiles: configuration 13, whose 128 X
//    rows cover M (a 256x256 tile would spend half its MFMAs on zero rows);
//  - else half a round of 256x128 tiles (configuration 13: 256 W rows, 128 X
//    rows), else half a round of 128x128 tiles (configuration 15, two
//    workgroups per CU);
//  - else (fewer than 128 tiles even at 128x128): the 128x128 ring tile
//    (configuration 3), or for M <= 256 the 128x64 ring tile (configuration
//    4), with the K range split so that the units fill at most one workgroup
//    per CU (2 to 4 splits of at least 8 k-tiles, when K has at least 32).
//    Sustained: 512x9728x2560 three ways 36.4 us against 38.7 for the
//    register-staged 128x128 tile (configuration 15) and 40.8 two ways;
//    256x3072x3072 at 128x64 split two ways 15.6 us against 17.2-18.5 for
//    128x128 split two to four ways, and 16.3 with a 6-stage ring.  More
//    splits lose to the partial-sum traffic, stream-K to its bookkeeping;
//  - M <= 64: the W-streaming ring tiles with a short X tile.
// A host-side grid mode: the whole rounds of a tile grid, then the last
// round's tiles split two ways along K (count: the tiles done whole).
constexpr int kGridSplitTail = 8;

TileChoice choose_tiles(int64_t M, int64_t N, int64_t K, int epi = INV_EPI_NONE) {
    TileChoice c{17, inv::GRID_TILES, 1};
    const int cus = g.cu_count > 0 ? g.cu_count : 256;
    auto tiles_of = [&](int cfg) { return ((M + kCfg[cfg].tm - 1) / kCfg[cfg].tm) * ((N + kCfg[cfg].tn - 1) / kCfg[cfg].tn); };
    if (M <= 32) {
        c.cfg = 5;
    } else if (M <= 64) {
        c.cfg = 4;
    } else if (M <= 128 && tiles_of(13) * 2 >= cus) {
        c.cfg = 13;  // 128 X rows cover M: a 256-row tile would multiply zeros for half its MFMAs
    } else if (tiles_of(17) * 4 >= (int64_t)cus * 3) {
        // 256x256 tiles of 8 waves (17) or 256x224 of 4 waves (16), whichever leaves fewer
        // CUs idle in the last round and fewer MFMAs on zero padding at the edges; 17 runs a
        // full round about 10% faster (fitted over ten shapes: 0.93 to 1.16).
        auto score = [&](int cfg) {
            const int64_t tm = (M + kCfg[cfg].tm - 1) / kCfg[cfg].tm, tn = (N + kCfg[cfg].tn - 1) / kCfg[cfg].tn;
            const int64_t t = tm * tn, rounds = (t + cus - 1) / cus;
            return (double)t / (double)(rounds * cus) * (double)M / (double)(tm * kCfg[cfg].tm) * (double)N /
                   (double)(tn * kCfg[cfg].tn);
        };
        c.cfg = (score(16) > 1.10 * score(17)) ? 16 : 17;
        // 256x192 tiles (18) run a round ~10% less efficiently per FLOP than
        // 256x224 but can fill the last round where neither of the others does
        // (9216 x 3840 -> 3840: 720 tiles in 3 rounds against 630 in 2.46; 229
        // us against 241).  Not where 16's last round takes the split tail
        // (below), which fills it better (9216 x 15360 -> 3840: 885 against 921).
        const int64_t t16 = tiles_of(16), tail16 = t16 % cus, kt16 = (K + kCfg[16].bk - 1) / kCfg[16].bk;
        const bool tail_fills_16 = t16 > cus && tail16 > 0 && 2 * tail16 <= cus && kt16 >= 128;
        if (!tail_fills_16 && 0.90 * score(18) > std::max(score(16), 1.10 * score(17))) c.cfg = 18;
    } else if (tiles_of(13) * 2 >= cus) {
        c.cfg = 13;
    } else {
        c.cfg = (M <= 256) ? 4 : 3;
        const int64_t KT = (K + kCfg[c.cfg].bk - 1) / kCfg[c.cfg].bk;
        const int64_t ks = std::min<int64_t>({4, cus / tiles_of(c.cfg), KT / 8});
        if (KT >= 32 && ks >= 2) {
            c.mode = inv::GRID_SPLITK;
            c.count = (int)ks;
        }
    }
    int ov = env_int("INV_HIP_TILE_CFG", -1);
    if (ov >= 0 && ov < kNumCfg) c.cfg = ov;
    const CfgMeta &m = kCfg[c.cfg];
    const int64_t slots = (int64_t)cus * cfg_occupancy(m);
    const int mode = env_int("INV_HIP_MODE", -1);
    if (mode == inv::GRID_TILES) {
        c.mode = inv::GRID_TILES;
    } else if (mode == inv::GRID_SPLITK) {
        c.mode = inv::GRID_SPLITK;
        c.count = std::max(1, env_int("INV_HIP_KSPLIT", 2));
    } else if (mode == inv::GRID_STREAMK) {
        c.mode = inv::GRID_STREAMK;
        c.count = std::max(1, env_int("INV_HIP_SK_GRID", (int)slots));
    }
    if (epi == INV_EPI_SWIGLU) {
        // gate | up wave columns over 256-row tiles, one workgroup per tile
        if (!kCfg[c.cfg].swiglu_ok) c.cfg = (M > 128) ? 8 : 2;
        c.mode = inv::GRID_TILES;
    }
    // Split tail: a tile grid whose last round is at most half full, on a long
    // K, runs its whole rounds as tiles and then its last round's tiles split
    // two ways along K (twice the workgroups, half the loop each; their
    // partial sums summed in K order).  The second launch and the partial sums
    // cost about what the half round saves at K = 3840 on the 256x224 tiles
    // (9216 x 3840 -> 3840: 253 us against 248 whole), and a little less on
    // the 8-wave 256x256 ones (-> 11520: 672 against 681; -> 15360: 912
    // against 930), so it is taken from 128 k-tiles (9216 x 15360 -> 3840: 912
    // us against 986), or from 60 on configuration 17.
    // INV_HIP_SPLIT_TAIL=0 turns it off; INV_HIP_SPLIT_TAIL_SLOTS sets the
    // slots per round and lifts the K limit (tests).
    const int64_t sl = env_int("INV_HIP_SPLIT_TAIL_SLOTS", 0) > 0 ? env_int("INV_HIP_SPLIT_TAIL_SLOTS", 0) : slots;
    const int64_t nt = tiles_of(c.cfg), tail = nt % sl, KT = (K + m.bk - 1) / m.bk;
    const int64_t min_kt = env_int("INV_HIP_SPLIT_TAIL_SLOTS", 0) > 0 ? 16 : (c.cfg == 17 ? 60 : 128);
    if (c.mode == inv::GRID_TILES && mode < 0 && epi != INV_EPI_SWIGLU && kCfg[c.cfg].staged_epi &&
        env_int("INV_HIP_SPLIT_TAIL", 1) && nt > sl && tail > 0 && 2 * tail <= sl && KT >= min_kt) {
        c.mode = kGridSplitTail;
        c.count = (int)(nt - tail);
    }
    return c;
}

// W [N x ldw], X [M x ldx] bf16 device; K a multiple of 8 (zero padded).
// Caller-provided split-K workspace in ordinary device memory (the
// no-allocation entry point's scratch): partial sums and arrival counters,
// the counters zero on entry.
struct FixedWorkspace {
    float *partial;
    size_t partial_bytes;
    unsigned *counters;
    size_t counter_bytes;
};

int run_gemm(const uint16_t *W, int64_t ldw, const uint16_t *X, int64_t ldx, void *Y, int64_t ldy, int out,
             const float *bias, const float *Cin, int64_t ldc, float alpha, float beta, int64_t M, int64_t N,
             int64_t K, int epi, int64_t w_seg_k = 0, int64_t Kw = -1, int64_t nout = -1,
             const float *colscale = nullptr, const float *row_bias = nullptr,
             const FixedWorkspace *fixed_ws = nullptr, const TileChoice *tiles = nullptr) {
    if (M == 0 || N == 0) return INV_OK;
    if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2) return fail(INV_ERR_ARG, "dimension too large");
    if (K % 8 || ldw % 8 || ldx % 8 || !aligned(W, 16) || !aligned(X, 16))
        return fail(INV_ERR_ARG, "internal: GEMM operands not 16-byte granular");
    if ((int64_t)256 * ldw * 2 >= ((int64_t)1 << 31) || (int64_t)256 * ldx * 2 >= ((int64_t)1 << 31))
        return fail(INV_ERR_UNSUPPORTED, "leading dimension too large for 32-bit buffer offsets");
    // tiles: a choice made by the caller (a row band of a larger product runs
    // the whole product's tiles); else the choice for this M.
    const TileChoice tc = tiles ? *tiles : choose_tiles(M, N, K, epi);
    if (epi == INV_EPI_SWIGLU && beta != 0.0f) return fail(INV_ERR_UNSUPPORTED, "SwiGLU epilogue with beta != 0");
    if (row_bias && (epi != INV_EPI_NONE || !kCfg[tc.cfg].staged_epi))
        return fail(INV_ERR_UNSUPPORTED, "internal: a per-row bias needs the staged epilogue and no activation");
    inv::GemmParams p{};
    p.nout = (int)(nout < 0 ? N : nout);
    p.W = W;
    p.X = X;
    p.Y = Y;
    p.bias = bias;
    p.Cin = Cin;
    p.ldw = ldw;
    p.ldx = ldx;
    p.ldy = ldy;
    p.ldc = ldc;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.w_seg_k = (int)w_seg_k;
    p.Kw = (int)(Kw < 0 ? K : Kw);
    const CfgMeta &cm = kCfg[tc.cfg];
    p.tiles_m = (int)((M + cm.tm - 1) / cm.tm);
    p.tiles_n = (int)((N + cm.tn - 1) / cm.tn);
    p.group_m = std::max(1, std::min(p.tiles_m, env_int("INV_HIP_GROUP_M", 8)));
    p.alpha = alpha;
    p.beta = beta;
    p.has_bias = bias != nullptr;
    p.colscale = colscale;
    p.row_bias = row_bias;
    const size_t esz = (out == inv::OUT_F32) ? 4 : 2;
    p.vec_store = (ldy % 4 == 0) && aligned(Y, 4 * esz) && (bias == nullptr || aligned(bias, 16));
    if (bias && !aligned(bias, 16)) return fail(INV_ERR_ARG, "internal: bias not 16-byte aligned");
    const int64_t KT = (K + cm.bk - 1) / cm.bk;  // the kernel's k-tiles
    const int64_t ntiles = (int64_t)p.tiles_m * p.tiles_n;
    int mode = tc.mode, count = tc.count;
    p.ksplit = 1;
    p.kt_per_split = (int)KT;
    // Split tail: tiles 0 .. dp_tiles-1 in a tile launch, the rest split two ways.
    int64_t dp_tiles = 0;
    if (mode == kGridSplitTail && fixed_ws &&
        (size_t)((ntiles - std::min<int64_t>(count, ntiles - 1)) * 2 * cm.threads * cm.acc_regs) * sizeof(float) >
            fixed_ws->partial_bytes)
        mode = inv::GRID_TILES;  // a caller's scratch too small for the split tail: the plain grid
    if (mode == kGridSplitTail) {
        dp_tiles = std::max<int64_t>(0, std::min<int64_t>(count, ntiles - 1));
        p.tile_base = (int)dp_tiles;
        p.tile_count = (int)(ntiles - dp_tiles);
        mode = inv::GRID_SPLITK;
        count = 2;
    }
    if (mode == inv::GRID_SPLITK) {
        p.kt_per_split = (int)((KT + count - 1) / count);
        p.ksplit = (int)((KT + p.kt_per_split - 1) / p.kt_per_split);
        if (p.ksplit <= 1) {
            mode = inv::GRID_TILES;
            p.ksplit = 1;
            p.kt_per_split = (int)KT;
        }
    } else if (mode == inv::GRID_STREAMK) {
        // Whole rounds except the last full one go one tile per workgroup;
        // the last full round plus the remainder are balanced, so each
        // workgroup's balanced share is at least one tile's K loop.
        const int64_t G = std::min<int64_t>(tc.count, ntiles * KT);
        int64_t dp_rounds = std::max<int64_t>(0, ntiles / G - 1);
        const int ov_rounds = env_int("INV_HIP_SK_DP_ROUNDS", -1);
        if (ov_rounds >= 0) dp_rounds = std::min<int64_t>(ov_rounds, ntiles / G);
        const int64_t rest = (ntiles - dp_rounds * G) * KT;  // k-iterations of the balanced phase
        p.ksplit = (int)(rest > 0 ? std::min<int64_t>(G, rest) : G);  // persistent grid size
        p.sk_dp_tiles = (int)(dp_rounds * G);
    }
    if (mode != inv::GRID_TILES) {
        const int64_t slots = (mode == inv::GRID_SPLITK) ? (p.tile_count > 0 ? p.tile_count : ntiles) * p.ksplit
                                                          : 2 * (int64_t)p.ksplit;
        const size_t pbytes = (size_t)(slots * cm.threads * cm.acc_regs) * sizeof(float);
        const size_t cbytes = (size_t)ntiles * sizeof(unsigned);
        if (fixed_ws) {
            if (pbytes > fixed_ws->partial_bytes || cbytes > fixed_ws->counter_bytes)
                return fail(INV_ERR_UNSUPPORTED,
                            "split-K needs %zu bytes of partial sums and %zu of counters; the no-allocation "
                            "scratch (%d MiB) has %zu and %zu left", pbytes, cbytes,
                            (int)(INV_NOALLOC_SCRATCH_BYTES >> 20), fixed_ws->partial_bytes, fixed_ws->counter_bytes);
            p.partial = fixed_ws->partial;
            p.counters = fixed_ws->counters;
            p.ws_cached = 1;
            // The counters start at zero (a fill kernel, not a memset node, so
            // the call may be captured into a graph).
            const int64_t nc = (int64_t)(cbytes / sizeof(unsigned));
            hipLaunchKernelGGL(fill_zero_u32, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, g.stream, p.counters,
                               nc);
            HIPCHK(hipGetLastError());
        } else {
            TRY(ensure_uncached(g.partial, pbytes, false));
            TRY(ensure_uncached(g.counters, cbytes, true));
            p.partial = (float *)g.partial.p;
            p.counters = (unsigned *)g.counters.p;
            p.ws_cached = 0;
        }
    }
    if (g.stats) HIPCHK(hipEventRecord(g.st0, g.stream));
    if (dp_tiles > 0) {  // the whole rounds, before the split tail
        inv::GemmParams pd = p;
        pd.tile_base = 0;
        pd.tile_count = (int)dp_tiles;
        pd.ksplit = 1;
        pd.kt_per_split = (int)KT;
        HIPCHK(cm.launch(pd, row_bias ? inv::EPI_ROWBIAS : epi, out, inv::GRID_TILES, g.stream));
    }
    HIPCHK(cm.launch(p, row_bias ? inv::EPI_ROWBIAS : epi, out, mode, g.stream));
    if (g.stats) {
        HIPCHK(hipEventRecord(g.st1, g.stream));
        HIPCHK(hipEventSynchronize(g.st1));
        float ms = 0.f;
        HIPCHK(hipEventElapsedTime(&ms, g.st0, g.st1));
        g.gemm_ms += ms;
        g.flops += 2.0 * (double)M * (double)N * (double)K;
    }
    return INV_OK;
}

int launch_cvt_rows_f32(const float *src, int64_t lds, uint16_t *dst, int64_t ldd, int64_t rows, int64_t cols,
                        int64_t cols_pad, int nseg = 1, int lo_mask = 0) {
    if (rows == 0) return INV_OK;
    int64_t work = rows * (cols_pad / 8);
    int vec = aligned(src, 16) && (lds % 4 == 0);
    hipLaunchKernelGGL(inv::cvt_rows_f32_bf16, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, g.stream, src, lds,
                       dst, ldd, rows, cols, cols_pad, vec, nseg, lo_mask);
    HIPCHK(hipGetLastError());
    return INV_OK;
}

int launch_copy_rows_bf16(const uint16_t *src, int64_t lds, uint16_t *dst, int64_t ldd, int64_t rows, int64_t cols,
                          int64_t cols_pad) {
    if (rows == 0) return INV_OK;
    int64_t work = rows * (cols_pad / 8);
    hipLaunchKernelGGL(inv::copy_rows_bf16, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, g.stream, src, lds,
                       dst, ldd, rows, cols, cols_pad);
    HIPCHK(hipGetLastError());
    return INV_OK;
}

// src [rows x cols] -> dst [cols x rows_pad] bf16
template <typename T>
int launch_transpose(const T *src, int64_t lds, uint16_t *dst, int64_t ldd, int64_t rows, int64_t cols,
                     int64_t rows_pad, int nseg = 1, int lo_mask = 0) {
    if (rows_pad == 0 || cols == 0) return INV_OK;
    dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows_pad + 63) / 64));
    if (grid.y > 65535) return fail(INV_ERR_UNSUPPORTED, "transpose: too many rows");
    const bool vec = nseg == 1 && cols % 64 == 0 && rows_pad % 64 == 0 && aligned(src, 16) &&
                     lds % (16 / (int64_t)sizeof(T)) == 0 && aligned(dst, 16) && ldd % 8 == 0;
    if (vec)
        hipLaunchKernelGGL(inv::transpose64_to_bf16<T>, grid, dim3(256), 0, g.stream, src, lds, dst, ldd, rows,
                           rows_pad);
    else
        hipLaunchKernelGGL(inv::transpose_to_bf16<T>, grid, dim3(256), 0, g.stream, src, lds, dst, ldd, rows, cols,
                           rows_pad, nseg, lo_mask);
    HIPCHK(hipGetLastError());
    return INV_OK;
}

int check_init() {
    if (!g.init) return fail(INV_ERR_NOT_INIT, "inv_hip_init has not been called (or failed)");
    HIPCHK(hipSetDevice(g.device));
    return INV_OK;
}

bool valid_weight(inv_weight_t w) {
    if (!w) return false;
    for (auto *x : g.weights)
        if (x == w) return w->magic == kWeightMagic;
    return false;
}

int epi_ok(int epi) {
    return epi == INV_EPI_NONE || epi == INV_EPI_SILU || epi == INV_EPI_GELU_ERF || epi == INV_EPI_SWIGLU;
}

int upload_bias(const float *bias, int64_t N, float **out) {
    *out = nullptr;
    if (!bias) return INV_OK;
    float *d = nullptr;
    TRY(dev_alloc((void **)&d, (size_t)N * 4, "bias"));
    int rc = h2d_rows(d, bias, 1, (size_t)N * 4, (size_t)N * 4);
    if (rc) {
        dev_free(d);
        return rc;
    }
    *out = d;
    return INV_OK;
}

int weight_upload_impl(const void *w, bool is_f32, int64_t N, int64_t K, const float *bias, inv_weight_t *out) {
    TRY(check_init());
    if (!out) return fail(INV_ERR_ARG, "out handle pointer is null");
    *out = nullptr;
    if (!w || N <= 0 || K <= 0) return fail(INV_ERR_ARG, "weight: null pointer or non-positive shape (N=%lld K=%lld)",
                                            (long long)N, (long long)K);
    if (N > INT32_MAX / 2 || K > INT32_MAX / 2) return fail(INV_ERR_ARG, "weight too large");
    const int64_t ldw = round_up(K, 8);
    uint16_t *dw = nullptr;
    TRY(dev_alloc((void **)&dw, (size_t)(N * ldw) * 2, "weight"));
    int rc = INV_OK;
    if (is_f32 && (size_t)ldw * 2 <= kPinChunk) {  // rounded by the host on its way up
        rc = h2d_rows_bf16(dw, (const float *)w, N, K, K, ldw);
    } else if (is_f32) {
        rc = ensure(g.win, (size_t)(N * K) * 4);
        if (!rc) rc = h2d_rows(g.win.p, w, N, (size_t)K * 4, (size_t)K * 4);
        if (!rc) rc = launch_cvt_rows_f32((const float *)g.win.p, K, dw, ldw, N, K, ldw);
    } else if (ldw == K) {
        rc = h2d_rows(dw, w, N, (size_t)K * 2, (size_t)K * 2);
    } else {
        rc = ensure(g.win, (size_t)(N * K) * 2);
        if (!rc) rc = h2d_rows(g.win.p, w, N, (size_t)K * 2, (size_t)K * 2);
        if (!rc) rc = launch_copy_rows_bf16((const uint16_t *)g.win.p, K, dw, ldw, N, K, ldw);
    }
    float *db = nullptr;
    if (!rc) rc = upload_bias(bias, N, &db);
    if (!rc) {
        hipError_t e = hipStreamSynchronize(g.stream);
        if (e != hipSuccess) rc = fail(INV_ERR_HIP, "weight upload: %s", hipGetErrorString(e));
    }
    if (rc) {
        dev_free(dw);
        dev_free(db);
        return rc;
    }
    auto *h = new inv_weight_s{kWeightMagic, dw, db, N, K, ldw, 0, N};
    g.weights.push_back(h);
    *out = h;
    return INV_OK;
}

size_t weight_bytes(const inv_weight_s *w) {
    return (size_t)(w->rows * w->ldw) * 2 + (w->bias ? (size_t)w->rows * 4 : 0);
}

void free_weight(inv_weight_s *w);

// Free a handle the library still lists (g.weights).
void drop_weight(inv_weight_s *w) {
    auto it = std::find(g.weights.begin(), g.weights.end(), w);
    if (it != g.weights.end()) g.weights.erase(it);
    free_weight(w);
}

// Evict least-recently-used cache entries nobody references until the cache
// fits its budget (entries in use are never evicted).
void cache_trim() {
    if (g.cache_budget <= 0) return;
    while (g.cache_bytes > (size_t)g.cache_budget) {
        int victim = -1;
        for (size_t i = 0; i < g.cache.size(); ++i)
            if (g.cache[i].w->refs == 0 && (victim < 0 || g.cache[i].last_use < g.cache[(size_t)victim].last_use))
                victim = (int)i;
        if (victim < 0) return;
        (void)hipStreamSynchronize(g.stream);
        g.cache_bytes -= g.cache[(size_t)victim].bytes;
        drop_weight(g.cache[(size_t)victim].w);
        g.cache.erase(g.cache.begin() + victim);
    }
}

// The cache key: the file's identity (device, inode, size, modification time,
// so a rewritten file is not served from the cache) and its resolved path,
// the tensor and bias names and the load flags.
int cache_key(const char *path, const char *name, const char *bias_name, int flags, std::string *key) {
    struct stat st;
    if (stat(path, &st) != 0) return fail(INV_ERR_ARG, "weight cache: cannot stat %s", path);
    char real[PATH_MAX];
    if (!realpath(path, real)) return fail(INV_ERR_ARG, "weight cache: cannot resolve %s", path);
    char id[128];
    snprintf(id, sizeof id, "%llu:%llu:%lld:%lld.%09ld", (unsigned long long)st.st_dev, (unsigned long long)st.st_ino,
             (long long)st.st_size, (long long)st.st_mtim.tv_sec, (long)st.st_mtim.tv_nsec);
    *key = std::string(id) + '\n' + real + '\n' + name + '\n' + (bias_name ? bias_name : "") + '\n' +
           std::to_string(flags);
    return INV_OK;
}

void free_weight(inv_weight_s *w) {
    dev_free(w->w);
    dev_free(w->bias);
    w->magic = 0;
    delete w;
}

// Stage an operand as bf16 rows with K contiguous: [rows x nseg*cols_pad],
// cols_pad = cols rounded up to seg_align (a multiple of 8).  With nseg > 1
// (fp32 sources only) segment s holds the lo parts of a hi/lo bf16 split if bit
// s of lo_mask is set, the hi parts otherwise.
//  src: host or device; dtype f32/bf16; trans: src holds the operand
//  transposed ([cols x rows] with leading dimension ld).
int stage_operand(const void *src, int dtype, bool on_device, bool trans, int64_t rows, int64_t cols, int64_t ld,
                  int nseg, int lo_mask, int64_t seg_align, Buf &dst, Buf &tmp, const uint16_t **out,
                  int64_t *out_ld) {
    const size_t esz = dtype == INV_DT_F32 ? 4 : 2;
    const int64_t cols_pad = round_up(cols, seg_align);
    const int64_t row_w = nseg * cols_pad;
    const int64_t src_rows = trans ? cols : rows;
    const int64_t src_cols = trans ? rows : cols;
    if (dtype == INV_DT_BF16 && nseg != 1) return fail(INV_ERR_ARG, "internal: split of a bf16 operand");
    // bf16, not transposed, already 16-byte granular on the device: use in place.
    if (on_device && dtype == INV_DT_BF16 && !trans && cols == cols_pad && ld % 8 == 0 && aligned(src, 16)) {
        *out = (const uint16_t *)src;
        *out_ld = ld;
        return INV_OK;
    }
    const void *dsrc = src;
    int64_t dld = ld;
    if (!on_device) {
        // fp32 rounded plainly: by the host, on its way into the bounce buffers
        if (!trans && dtype == INV_DT_F32 && nseg == 1 && lo_mask == 0 && (size_t)cols_pad * 2 <= kPinChunk) {
            TRY(ensure(dst, (size_t)(rows * cols_pad) * 2));
            TRY(h2d_rows_bf16((uint16_t *)dst.p, (const float *)src, rows, cols, ld, cols_pad));
            *out = (const uint16_t *)dst.p;
            *out_ld = cols_pad;
            return INV_OK;
        }
        // Upload the exact extent into a contiguous device buffer.
        if (!trans && dtype == INV_DT_BF16 && cols == cols_pad) {
            TRY(ensure(dst, (size_t)(rows * cols_pad) * 2));
            TRY(h2d_rows(dst.p, src, rows, (size_t)cols * 2, (size_t)ld * esz));
            *out = (const uint16_t *)dst.p;
            *out_ld = cols_pad;
            return INV_OK;
        }
        TRY(ensure(tmp, (size_t)(src_rows * src_cols) * esz));
        TRY(h2d_rows(tmp.p, src, src_rows, (size_t)src_cols * esz, (size_t)ld * esz));
        dsrc = tmp.p;
        dld = src_cols;
    }
    TRY(ensure(dst, (size_t)(rows * row_w) * 2));
    uint16_t *d = (uint16_t *)dst.p;
    if (!trans) {
        if (dtype == INV_DT_F32)
            TRY(launch_cvt_rows_f32((const float *)dsrc, dld, d, row_w, rows, cols, cols_pad, nseg, lo_mask));
        else
            TRY(launch_copy_rows_bf16((const uint16_t *)dsrc, dld, d, row_w, rows, cols, cols_pad));
    } else {
        // dsrc is [cols x rows] (ld dld) -> d [rows x row_w]
        if (dtype == INV_DT_F32)
            TRY(launch_transpose<float>((const float *)dsrc, dld, d, row_w, cols, rows, cols_pad, nseg, lo_mask));
        else
            TRY(launch_transpose<uint16_t>((const uint16_t *)dsrc, dld, d, row_w, cols, rows, cols_pad, 1, 0));
    }
    *out = d;
    *out_ld = row_w;
    return INV_OK;
}

int gemm_slot(int order, int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const void *A,
              int64_t lda, const void *B, int64_t ldb, float beta, float *C, int64_t ldc, int dtype) {
    TRY(check_init());
    if (order == INV_CBLAS_COL_MAJOR) {
        // Column-major C = op(A) op(B)  <=>  row-major C^T = op(B)^T op(A)^T.
        std::swap(transA, transB);
        std::swap(M, N);
        std::swap(A, B);
        std::swap(lda, ldb);
        order = INV_CBLAS_ROW_MAJOR;
    }
    if (order != INV_CBLAS_ROW_MAJOR) return fail(INV_ERR_ARG, "sgemm: bad order %d", order);
    auto tr_ok = [](int t) { return t == INV_CBLAS_NO_TRANS || t == INV_CBLAS_TRANS; };
    if (!tr_ok(transA) || !tr_ok(transB)) return fail(INV_ERR_ARG, "sgemm: bad transpose flag");
    if (M < 0 || N < 0 || K < 0) return fail(INV_ERR_ARG, "sgemm: negative dimension");
    if (M == 0 || N == 0) return INV_OK;
    if (!C) return fail(INV_ERR_ARG, "sgemm: C is null");
    if (ldc < std::max<int64_t>(1, N)) return fail(INV_ERR_ARG, "sgemm: ldc < N");
    const bool ta = transA == INV_CBLAS_TRANS, tb = transB == INV_CBLAS_TRANS;
    // Row-major: op(A) is M x K (A is K x M when transposed); op(B) is K x N.
    if (K > 0) {
        if (!A || !B) return fail(INV_ERR_ARG, "sgemm: A or B is null");
        if (lda < std::max<int64_t>(1, ta ? M : K)) return fail(INV_ERR_ARG, "sgemm: lda too small");
        if (ldb < std::max<int64_t>(1, tb ? K : N)) return fail(INV_ERR_ARG, "sgemm: ldb too small");
    }
    if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2) return fail(INV_ERR_ARG, "sgemm: too large");
    const int64_t Kp = round_up(std::max<int64_t>(K, 1), 8);
    const uint16_t *Xd = nullptr, *Wd = nullptr;
    int64_t ldx = 0, ldw = 0;
    // Precision: fp32 operands are rounded to bf16 (1 pass), or split into
    // hi + lo and concatenated along K: A' = [Ah|Al], B' = [Bh|Bh] (2 passes)
    // or A' = [Ah|Al|Ah], B' = [Bh|Bh|Bl] (3 passes, ~fp32 accuracy).
    int nseg = 1, amask = 0, bmask = 0;
    if (dtype == INV_DT_F32) {
        if (g.sgemm_prec == INV_PREC_SPLIT_A) {
            nseg = 2;
            amask = 0x2;
        } else if (g.sgemm_prec == INV_PREC_SPLIT_AB) {
            nseg = 3;
            amask = 0x2;
            bmask = 0x4;
        }
    }
    int64_t Kgemm = nseg * Kp;
    if (K > 0) {
        // X = op(A) [M x K]: stored transposed when A is Trans.
        TRY(stage_operand(A, dtype, false, ta, M, K, lda, nseg, amask, 8, g.x16, g.xin, &Xd, &ldx));
        // W = op(B)^T [N x K]: B is [N x K] when Trans, [K x N] (transposed) otherwise.
        TRY(stage_operand(B, dtype, false, !tb, N, K, ldb, nseg, bmask, 8, g.w16, g.win, &Wd, &ldw));
    } else {
        Kgemm = 8;
        // K == 0: C = beta * C.  Zero operands of width 8.
        TRY(ensure(g.x16, (size_t)(M * 8) * 2));
        TRY(ensure(g.w16, (size_t)(N * 8) * 2));
        HIPCHK(hipMemsetAsync(g.x16.p, 0, (size_t)(M * 8) * 2, g.stream));
        HIPCHK(hipMemsetAsync(g.w16.p, 0, (size_t)(N * 8) * 2, g.stream));
        Xd = (const uint16_t *)g.x16.p;
        Wd = (const uint16_t *)g.w16.p;
        ldx = ldw = 8;
    }
    TRY(ensure(g.yout, (size_t)(M * N) * 4));
    const float *cin = nullptr;
    if (beta != 0.0f) {
        TRY(ensure(g.cin, (size_t)(M * N) * 4));
        TRY(h2d_rows(g.cin.p, C, M, (size_t)N * 4, (size_t)ldc * 4));
        cin = (const float *)g.cin.p;
    }
    TRY(run_gemm(Wd, ldw, Xd, ldx, g.yout.p, N, inv::OUT_F32, nullptr, cin, N, alpha, beta, M, N, Kgemm,
                 inv::EPI_NONE));
    TRY(d2h_rows(C, g.yout.p, M, (size_t)N * 4, (size_t)ldc * 4));
    g.calls++;
    return INV_OK;
}

// Y = epilogue(X . W^T + bias), or with accumulate Y += gate[n] * (X . W^T + bias)
// (gate null: a plain residual add).  Y stays fp32 when accumulating.
// A row normalisation applied while the fp32 X is rounded into the bf16 operand.
struct NormArgs {
    int kind;            // INV_NORM_ADALN or INV_NORM_RMS
    const float *scale;  // AdaLN scale (the 1 + scale factor) or RMS weight, [K]
    const float *shift;  // AdaLN shift [K]; null for RMS
    float eps;
};

// The normalisation's per-column vectors as the row kernels read them: host
// vectors uploaded, device vectors not 16-byte aligned copied (the register
// kernel reads them 16 bytes at a time); null stays null.
int stage_norm_vectors(const NormArgs &nm, bool dev, int64_t K, const float **ad, const float **bd) {
    *ad = nm.scale;
    *bd = nm.shift;
    const size_t vb = (size_t)K * 4;
    if (!dev) {
        TRY(ensure(g.nvec, 2 * vb));
        if (nm.scale) TRY(h2d_rows(g.nvec.p, nm.scale, 1, vb, vb));
        if (nm.shift) TRY(h2d_rows((char *)g.nvec.p + vb, nm.shift, 1, vb, vb));
    } else if ((*ad && !aligned(*ad, 16)) || (*bd && !aligned(*bd, 16))) {
        TRY(ensure(g.nvec, 2 * vb));
        if (*ad) HIPCHK(hipMemcpyAsync(g.nvec.p, *ad, vb, hipMemcpyDeviceToDevice, g.stream));
        if (*bd) HIPCHK(hipMemcpyAsync((char *)g.nvec.p + vb, *bd, vb, hipMemcpyDeviceToDevice, g.stream));
    } else {
        return INV_OK;
    }
    *ad = nm.scale ? (const float *)g.nvec.p : nullptr;
    *bd = nm.shift ? (const float *)((char *)g.nvec.p + vb) : nullptr;
    return INV_OK;
}

// d[M x ldw] bf16 = norm(xd[M x K] fp32) on the library stream, one workgroup
// per row (ad, bd from stage_norm_vectors).
int launch_norm_rows(const float *xd, const NormArgs &nm, const float *ad, const float *bd, int64_t M, int64_t K,
                     uint16_t *d, int64_t ldw) {
    if (M == 0) return INV_OK;
    const bool in_regs = K % 4 == 0 && K <= 4 * 256 * inv::NORM_ROW_GROUPS && aligned(xd, 16);
    if (in_regs) {
        const int64_t groups = (K / 4 + 255) / 256;  // register groups of 4 columns per thread
        auto launch = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3((unsigned)M), dim3(256), 0, g.stream, xd, K, ad, bd, nm.eps, d, ldw, K,
                               ldw);
        };
        const bool ada = nm.kind == INV_NORM_ADALN;
        using namespace inv;
#define INV_NORM_J(J) (ada ? launch(norm_rows_f32_bf16_reg<NORM_ADALN, J>) : launch(norm_rows_f32_bf16_reg<NORM_RMS, J>))
        if (groups <= 1) INV_NORM_J(1);
        else if (groups <= 2) INV_NORM_J(2);
        else if (groups <= 3) INV_NORM_J(3);
        else if (groups <= 4) INV_NORM_J(4);
        else if (groups <= 6) INV_NORM_J(6);
        else if (groups <= 8) INV_NORM_J(8);
        else if (groups <= 12) INV_NORM_J(12);
        else INV_NORM_J(16);
#undef INV_NORM_J
    } else if (nm.kind == INV_NORM_ADALN)
        hipLaunchKernelGGL(inv::norm_rows_f32_bf16<inv::NORM_ADALN>, dim3((unsigned)M), dim3(256), 0, g.stream, xd, K,
                           ad, bd, nm.eps, d, ldw, K, ldw);
    else
        hipLaunchKernelGGL(inv::norm_rows_f32_bf16<inv::NORM_RMS>, dim3((unsigned)M), dim3(256), 0, g.stream, xd, K,
                           ad, bd, nm.eps, d, ldw, K, ldw);
    HIPCHK(hipGetLastError());
    return INV_OK;
}

// Stage X = norm(X_f32) as bf16 [M x round_up(K, 8)] in g.x16 (X, scale and
// shift host or device per `dev`).
int stage_normalized(const char *who, const float *X, const NormArgs &nm, bool dev, int64_t M, int64_t K,
                     const uint16_t **out, int64_t *out_ld) {
    const int64_t ldw = round_up(K, 8);
    const float *xd = X;
    if (!dev) {
        TRY(ensure(g.xin, (size_t)(M * K) * 4));
        TRY(h2d_rows(g.xin.p, X, M, (size_t)K * 4, (size_t)K * 4));
        xd = (const float *)g.xin.p;
    } else if (!aligned(X, 4)) {
        return fail(INV_ERR_ARG, "%s: X not 4-byte aligned", who);
    }
    const float *ad = nullptr, *bd = nullptr;
    TRY(stage_norm_vectors(nm, dev, K, &ad, &bd));
    TRY(ensure(g.x16, (size_t)(M * ldw) * 2));
    uint16_t *d = (uint16_t *)g.x16.p;
    TRY(launch_norm_rows(xd, nm, ad, bd, M, K, d, ldw));
    *out = d;
    *out_ld = ldw;
    return INV_OK;
}

// Argument checks shared by the linear entry points (status, no side effects).
int check_linear_args(const char *who, int x_dtype, inv_weight_t W, int y_dtype, int64_t M, int64_t K, int64_t N,
                      int epilogue, int flags, bool accumulate, const float *bias) {
    if (!valid_weight(W)) return fail(INV_ERR_ARG, "%s: unknown weight handle", who);
    if (x_dtype != INV_DT_F32 && x_dtype != INV_DT_BF16) return fail(INV_ERR_ARG, "%s: bad x_dtype %d", who, x_dtype);
    if (y_dtype != INV_DT_F32 && y_dtype != INV_DT_BF16) return fail(INV_ERR_ARG, "%s: bad y_dtype %d", who, y_dtype);
    if (!epi_ok(epilogue)) return fail(INV_ERR_ARG, "%s: bad epilogue %d", who, epilogue);
    if (flags & ~(INV_FLAG_DEVICE_PTRS | INV_FLAG_ASYNC | INV_FLAG_PRECISE))
        return fail(INV_ERR_ARG, "%s: unknown flags 0x%x", who, flags);
    if ((flags & INV_FLAG_ASYNC) && !(flags & INV_FLAG_DEVICE_PTRS))
        return fail(INV_ERR_ARG, "%s: ASYNC requires DEVICE_PTRS", who);
    if (M < 0) return fail(INV_ERR_ARG, "%s: negative M", who);
    if (K != W->K || N != W->N)
        return fail(INV_ERR_ARG, "%s: shape mismatch: call K=%lld N=%lld, weight K=%lld N=%lld", who, (long long)K,
                    (long long)N, (long long)W->K, (long long)W->N);
    if (accumulate && W->gated) return fail(INV_ERR_ARG, "%s: a gate/up weight has no gated-add form", who);
    if ((epilogue == INV_EPI_SWIGLU) != (W->gated != 0))
        return fail(INV_ERR_ARG, W->gated ? "linear: a gate/up weight needs INV_EPI_SWIGLU"
                                          : "linear: INV_EPI_SWIGLU needs a gate/up weight (inv_hip_weight_upload_gate_up)");
    if (W->gated && bias) return fail(INV_ERR_ARG, "%s: a gate/up weight takes its biases at upload", who);
    if (M > INT32_MAX / 2) return fail(INV_ERR_ARG, "%s: M too large", who);
    return INV_OK;
}

// inv_hip_linear on device pointers with no allocation: activations staged,
// a misaligned bias copied and split-K partials parked in the library's
// static scratch array (g.scratch), whose split-K counters are cleared by a
// fill kernel before each GEMM that uses them.  Everything runs on the
// library stream, so successive calls never overlap.
int linear_noalloc_impl(const void *X, int x_dtype, inv_weight_t W, const float *bias, void *Y, int y_dtype,
                        int64_t M, int64_t K, int64_t N, int epilogue, int flags) {
    const char *who = "linear_noalloc";
    TRY(check_init());
    if (!g.scratch) return fail(INV_ERR_NOT_INIT, "%s: the scratch array has no device address", who);
    TRY(check_linear_args(who, x_dtype, W, y_dtype, M, K, N, epilogue, flags, false, bias));
    if (!(flags & INV_FLAG_DEVICE_PTRS))
        return fail(INV_ERR_ARG, "%s: needs INV_FLAG_DEVICE_PTRS (host pointers would need bounce buffers)", who);
    if (M == 0) return INV_OK;
    if (!X || !Y) return fail(INV_ERR_ARG, "%s: X or Y is null", who);
    const int out = (y_dtype == INV_DT_F32) ? inv::OUT_F32 : inv::OUT_BF16;
    unsigned char *const base = g.scratch;
    unsigned char *const stage = base + kScratchCounters + kScratchBias;
    const size_t stage_cap = INV_NOALLOC_SCRATCH_BYTES - kScratchCounters - kScratchBias;

    // Activations: bf16 rows [M x ldx] with K contiguous, zero padded.
    const bool precise = (flags & INV_FLAG_PRECISE) && x_dtype == INV_DT_F32;
    const int64_t kseg = precise ? round_up(K, 64) : W->ldw;
    const uint16_t *Xd = nullptr;
    int64_t ldx = 0;
    size_t used = 0;
    if (x_dtype == INV_DT_BF16 && K == W->ldw && aligned(X, 16)) {
        Xd = (const uint16_t *)X;
        ldx = K;
    } else {
        ldx = precise ? 2 * kseg : W->ldw;
        used = (size_t)round_up(M * ldx * 2, 256);
        if (used > stage_cap)
            return fail(INV_ERR_UNSUPPORTED, "%s: staging %lld x %lld activations needs %zu bytes, above the %d MiB "
                        "no-allocation scratch", who, (long long)M, (long long)K, used,
                        (int)(INV_NOALLOC_SCRATCH_BYTES >> 20));
        uint16_t *d = (uint16_t *)stage;
        if (x_dtype == INV_DT_F32) {
            if (!aligned(X, 4)) return fail(INV_ERR_ARG, "%s: fp32 X not 4-byte aligned", who);
            TRY(launch_cvt_rows_f32((const float *)X, K, d, ldx, M, K, precise ? kseg : W->ldw, precise ? 2 : 1,
                                    precise ? 0x2 : 0));
        } else {
            if (!aligned(X, 2)) return fail(INV_ERR_ARG, "%s: bf16 X not 2-byte aligned", who);
            TRY(launch_copy_rows_bf16((const uint16_t *)X, K, d, ldx, M, K, W->ldw));
        }
        Xd = d;
    }

    // Bias: explicit argument first, else the handle's; 16-byte aligned for the epilogue.
    const float *bd = W->bias;
    if (bias) {
        if (aligned(bias, 16)) {
            bd = bias;
        } else {
            if ((size_t)N * 4 > kScratchBias)
                return fail(INV_ERR_UNSUPPORTED, "%s: a misaligned bias of %lld columns exceeds the scratch's bias "
                            "area", who, (long long)N);
            HIPCHK(hipMemcpyAsync(base + kScratchCounters, bias, (size_t)N * 4, hipMemcpyDeviceToDevice, g.stream));
            bd = (const float *)(base + kScratchCounters);
        }
    }
    const FixedWorkspace ws{(float *)(stage + used), stage_cap - used, (unsigned *)base, kScratchCounters};
    if (precise)
        TRY(run_gemm(W->w, W->ldw, Xd, ldx, Y, N, out, bd, nullptr, N, 1.0f, 0.0f, M, W->rows, 2 * kseg, epilogue,
                     kseg, W->ldw, N, nullptr, nullptr, &ws));
    else
        TRY(run_gemm(W->w, W->ldw, Xd, ldx, Y, N, out, bd, nullptr, N, 1.0f, 0.0f, M, W->rows, W->ldw, epilogue, 0,
                     -1, N, nullptr, nullptr, &ws));
    g.calls++;
    if (!(flags & INV_FLAG_ASYNC)) HIPCHK(hipStreamSynchronize(g.stream));
    return INV_OK;
}

// The band pipeline's streams, events and output bounce buffers, made on first
// use.  False (and the serial path is taken) when they cannot be made.
bool pipe_ready() {
    auto &P = g.pipe;
    if (P.tried) return P.ready;
    P.tried = true;
    bool ok = hipStreamCreateWithFlags(&P.up, hipStreamNonBlocking) == hipSuccess &&
              hipStreamCreateWithFlags(&P.down, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&P.start, hipEventDisableTiming) == hipSuccess;
    for (int k = 0; k < 2 && ok; ++k) {
        for (hipEvent_t *e : {&P.in_ev[k], &P.gemm_ev[k], &P.out_ev[k]})
            ok = ok && hipEventCreateWithFlags(e, hipEventDisableTiming) == hipSuccess &&
                 hipEventRecord(*e, P.up) == hipSuccess;  // complete before first use
        ok = ok && hipHostMalloc(&P.pin_out[k], kPinChunk, hipHostMallocDefault) == hipSuccess;
    }
    if (!ok) (void)hipGetLastError();
    P.ready = ok;
    return ok;
}

void release_pipe() {
    auto &P = g.pipe;
    for (hipStream_t s : {P.up, P.down})
        if (s) (void)hipStreamSynchronize(s);
    for (int k = 0; k < 2; ++k) {
        if (P.pin_out[k]) (void)hipHostFree(P.pin_out[k]);
        for (hipEvent_t e : {P.in_ev[k], P.gemm_ev[k], P.out_ev[k]})
            if (e) (void)hipEventDestroy(e);
    }
    if (P.start) (void)hipEventDestroy(P.start);
    for (hipStream_t s : {P.up, P.down})
        if (s) (void)hipStreamDestroy(s);
    P = {};
}

// Rows per band for a host-pointer projection, or 0 for one serial pass:
// about M / INV_HIP_HOST_BANDS (default 8) rows in whole tile rows, but at
// least ~16 MB of PCIe traffic per band, and fewer rows when a band's upload
// (up_row bytes per row: its X rows, and its Y rows when Y is accumulated) or
// download would not fit one bounce buffer (INV_HIP_HOST_BAND_MB caps the
// larger side below that).  Larger bands leave more of the first upload and the last
// download exposed; smaller ones pay ~80 us of host synchronisation, copy
// dispatch and launches per band, and a part-filled GEMM.  Measured with fp32
// X and Y (ms; one serial pass in brackets): 4608x3072 -> 9216 3.75 (5.01),
// 4608x3072 -> 3072 1.83 (2.54), 4608x12288 -> 3072 4.86 (5.86), 2048x3840 ->
// 15360 2.81 (3.46), 1024x3072 -> 3072 0.62 (0.73).  Only the one-launch tile
// grid is banded: its elements do not depend on M, so each band gives the bits
// one launch over all rows gives.
int64_t host_band_rows(int64_t tm, int64_t M, size_t up_row, size_t out_row) {
    const size_t cap = std::min(kPinChunk, (size_t)std::max(1, env_int("INV_HIP_HOST_BAND_MB", 32)) << 20);
    const int64_t bands = std::max(2, env_int("INV_HIP_HOST_BANDS", 8));
    const int64_t fit = (int64_t)(cap / std::max(up_row, out_row)) / tm * tm;
    const int64_t min_rows = round_up((int64_t)((16u << 20) / (up_row + out_row)) + 1, tm);
    const int64_t mb = std::min(fit, std::max(min_rows, M / bands / tm * tm));
    return (mb > 0 && M > mb) ? mb : 0;
}
int64_t host_band_rows(const TileChoice &tc, int64_t M, size_t up_row, size_t out_row) {
    return tc.mode == inv::GRID_TILES ? host_band_rows(kCfg[tc.cfg].tm, M, up_row, out_row) : 0;
}

// The row-band pipeline's optional stages: X normalised (fp32 X; the
// vectors already on the device), and Y accumulated (Y += gate * (...), Y
// uploaded band by band as well).
struct BandExtras {
    const NormArgs *nm = nullptr;
    const float *nscale = nullptr, *nshift = nullptr;
    bool accumulate = false;
    const float *gate = nullptr;  // device, or null
};

// The row-band pipeline's schedule, shared by the host-pointer entry points:
// rows [0, M) in bands of mb.  stage(r0, nr, pin) copies band rows from the
// host into the pinned buffer pin (band b uses pin[b & 1]) and queues their
// uploads on the `up` stream; compute(r0, nr) queues the band's kernels on the
// library stream, after those uploads; then the band's output, nr rows of
// out_row bytes at dev_out + r0 * out_row, goes down through pin_out[b & 1] to
// Y + r0 * out_row.  Band b+2 is staged and computed while band b drains, so
// upload, kernels and download of neighbouring bands overlap.  Returns when Y
// is written.
int run_band_pipeline(int64_t M, int64_t mb, char *Y, size_t out_row, const char *dev_out,
                      const std::function<int(int64_t, int64_t, char *)> &stage,
                      const std::function<int(int64_t, int64_t)> &compute) {
    auto &P = g.pipe;
    // The copy streams start after the library stream's earlier work (which
    // may still read the device buffers), and the bounce buffers after their uploads.
    HIPCHK(hipEventRecord(P.start, g.stream));
    HIPCHK(hipStreamWaitEvent(P.up, P.start, 0));
    HIPCHK(hipStreamWaitEvent(P.down, P.start, 0));
    for (int k = 0; k < 2; ++k) HIPCHK(hipEventSynchronize(g.pin_ev[k]));
    const int64_t nb = (M + mb - 1) / mb;
    auto rows_of = [&](int64_t b) { return std::min(mb, M - b * mb); };
    auto upload_and_compute = [&](int64_t b) -> int {
        const int k = (int)(b & 1);
        HIPCHK(hipEventSynchronize(P.in_ev[k]));  // band b-2's upload has left pin[k]
        TRY(stage(b * mb, rows_of(b), (char *)g.pin[k]));
        HIPCHK(hipEventRecord(P.in_ev[k], P.up));
        HIPCHK(hipStreamWaitEvent(g.stream, P.in_ev[k], 0));
        TRY(compute(b * mb, rows_of(b)));
        HIPCHK(hipEventRecord(P.gemm_ev[k], g.stream));
        return INV_OK;
    };
    auto download = [&](int64_t b) -> int {  // pin_out[b & 1] is free (band b-2 drained)
        const int k = (int)(b & 1);
        HIPCHK(hipStreamWaitEvent(P.down, P.gemm_ev[k], 0));
        HIPCHK(hipMemcpyAsync(P.pin_out[k], dev_out + (size_t)(b * mb) * out_row, (size_t)rows_of(b) * out_row,
                              hipMemcpyDeviceToHost, P.down));
        HIPCHK(hipEventRecord(P.out_ev[k], P.down));
        return INV_OK;
    };
    auto drain = [&](int64_t b) -> int {
        const int k = (int)(b & 1);
        HIPCHK(hipEventSynchronize(P.out_ev[k]));
        par_copy_rows(Y + (size_t)(b * mb) * out_row, out_row, (const char *)P.pin_out[k], out_row, rows_of(b),
                      out_row);
        return INV_OK;
    };
    auto run = [&]() -> int {
        for (int64_t b = 0; b < std::min<int64_t>(2, nb); ++b) TRY(upload_and_compute(b));
        for (int64_t b = 0; b < std::min<int64_t>(2, nb); ++b) TRY(download(b));
        for (int64_t b = 0; b < nb; ++b) {
            if (b + 2 < nb) TRY(upload_and_compute(b + 2));
            TRY(drain(b));
            if (b + 2 < nb) TRY(download(b + 2));
        }
        return INV_OK;
    };
    const int rc = run();
    if (rc != INV_OK) {
        // copies still in flight must not outlive the call: the bounce buffers
        // are reused by the next one
        (void)hipStreamSynchronize(P.up);
        (void)hipStreamSynchronize(g.stream);
        (void)hipStreamSynchronize(P.down);
    }
    return rc;
}

// Y = X W^T (+ bias, activation) with X and Y in host memory, in row bands of
// mb rows through run_band_pipeline: a band's conversion (or normalisation)
// and GEMM run while its neighbours upload and download.  When Y is
// accumulated, a band's Y rows travel up behind its X rows in the same bounce
// buffer.  Every band runs the tile choice tc of the whole product.
int linear_host_banded(const void *X, int x_dtype, inv_weight_t W, const float *bd, void *Y, int y_dtype, int64_t M,
                       int64_t K, int64_t N, int epilogue, const TileChoice &tc, int64_t mb, const BandExtras &ex) {
    const size_t xsz = (x_dtype == INV_DT_F32) ? 4 : 2, ysz = (y_dtype == INV_DT_F32) ? 4 : 2;
    const int out = (y_dtype == INV_DT_F32) ? inv::OUT_F32 : inv::OUT_BF16;
    const int64_t ldw = W->ldw;
    const size_t out_row = (size_t)N * ysz;
    // fp32 rows (not normalised) are rounded by the host into bf16 operand
    // rows; bf16 rows already 16-byte granular land in the operand as they are
    const bool host_round = !ex.nm && x_dtype == INV_DT_F32;
    const bool direct = host_round || (!ex.nm && x_dtype == INV_DT_BF16 && K == ldw);
    const size_t in_row = (size_t)K * xsz, up_row = host_round ? (size_t)ldw * 2 : in_row;
    TRY(ensure(g.x16, (size_t)(M * ldw) * 2));
    if (!direct) TRY(ensure(g.xin, (size_t)M * in_row));
    TRY(ensure(g.yout, (size_t)M * out_row));
    auto stage = [&](int64_t r0, int64_t nr, char *pin) -> int {
        char *yb = (char *)g.yout.p + (size_t)r0 * out_row;
        if (host_round)
            par_cvt_rows((uint16_t *)pin, ldw, (const float *)X + r0 * K, K, nr, K, ldw);
        else
            par_copy_rows(pin, in_row, (const char *)X + r0 * in_row, in_row, nr, in_row);
        if (ex.accumulate) par_copy_rows(pin + nr * up_row, out_row, (const char *)Y + r0 * out_row, out_row, nr, out_row);
        char *dst = direct ? (char *)g.x16.p + (size_t)r0 * ldw * 2 : (char *)g.xin.p + (size_t)r0 * in_row;
        HIPCHK(hipMemcpyAsync(dst, pin, (size_t)nr * up_row, hipMemcpyHostToDevice, g.pipe.up));
        if (ex.accumulate)
            HIPCHK(hipMemcpyAsync(yb, pin + nr * up_row, (size_t)nr * out_row, hipMemcpyHostToDevice, g.pipe.up));
        return INV_OK;
    };
    auto compute = [&](int64_t r0, int64_t nr) -> int {
        char *yb = (char *)g.yout.p + (size_t)r0 * out_row;
        uint16_t *xb = (uint16_t *)g.x16.p + r0 * ldw;
        if (ex.nm) {
            TRY(launch_norm_rows((const float *)g.xin.p + r0 * K, *ex.nm, ex.nscale, ex.nshift, nr, K, xb, ldw));
        } else if (!direct) {  // bf16 rows re-pitched to ldw
            TRY(launch_copy_rows_bf16((const uint16_t *)g.xin.p + r0 * K, K, xb, ldw, nr, K, ldw));
        }
        // accumulating reads the band's Y as C (beta = 1) in place, as the one-pass call does
        return run_gemm(W->w, ldw, xb, ldw, yb, N, out, bd, ex.accumulate ? (const float *)yb : nullptr, N, 1.0f,
                        ex.accumulate ? 1.0f : 0.0f, nr, W->rows, ldw, epilogue, 0, -1, N, ex.gate, nullptr, nullptr,
                        &tc);
    };
    TRY(run_band_pipeline(M, mb, (char *)Y, out_row, (const char *)g.yout.p, stage, compute));
    g.calls++;
    return INV_OK;
}

int linear_impl(const char *who, const void *X, int x_dtype, inv_weight_t W, const float *bias, void *Y, int y_dtype,
                int64_t M, int64_t K, int64_t N, int epilogue, int flags, bool accumulate, const float *gate,
                const NormArgs *nm = nullptr) {
    TRY(check_init());
    TRY(check_linear_args(who, x_dtype, W, y_dtype, M, K, N, epilogue, flags, accumulate, bias));
    if (M == 0) return INV_OK;
    if (!X || !Y) return fail(INV_ERR_ARG, "%s: X or Y is null", who);
    const bool dev = (flags & INV_FLAG_DEVICE_PTRS) != 0;
    const int out = (y_dtype == INV_DT_F32) ? inv::OUT_F32 : inv::OUT_BF16;
    const size_t ysz = (y_dtype == INV_DT_F32) ? 4 : 2;
    const bool precise = (flags & INV_FLAG_PRECISE) && x_dtype == INV_DT_F32;
    if (nm && precise) return fail(INV_ERR_UNSUPPORTED, "%s: INV_FLAG_PRECISE with a normalisation", who);

    // Bias: explicit argument first, else the handle's.
    const float *bd = W->bias;
    if (bias) {
        if (dev && aligned(bias, 16)) {
            bd = bias;
        } else {
            TRY(ensure(g.bias, (size_t)N * 4));
            if (dev)
                HIPCHK(hipMemcpyAsync(g.bias.p, bias, (size_t)N * 4, hipMemcpyDeviceToDevice, g.stream));
            else
                TRY(h2d_rows(g.bias.p, bias, 1, (size_t)N * 4, (size_t)N * 4));
            bd = (const float *)g.bias.p;
        }
    }

    // Gate: per-column scale of the projection (device pointers are used as
    // they are; a host gate is copied next to the bias).
    const float *gd = nullptr;
    if (accumulate && gate) {
        if (dev && aligned(gate, 4)) {
            gd = gate;
        } else {
            TRY(ensure(g.gate, (size_t)N * 4));
            if (dev)
                HIPCHK(hipMemcpyAsync(g.gate.p, gate, (size_t)N * 4, hipMemcpyDeviceToDevice, g.stream));
            else
                TRY(h2d_rows(g.gate.p, gate, 1, (size_t)N * 4, (size_t)N * 4));
            gd = (const float *)g.gate.p;
        }
    }

    // Host X and Y: the row-band pipeline (INV_HIP_HOST_PIPELINE: 0 never, 2
    // required: a host call it cannot take fails).
    if (!dev) {
        const int pipe_mode = env_int("INV_HIP_HOST_PIPELINE", 1);
        if (pipe_mode && !precise) {
            // bands run the whole product's tile grid, one launch each (a split
            // tail belongs to the whole grid's last round, not to a band's)
            TileChoice tc = choose_tiles(M, W->rows, W->ldw, epilogue);
            if (tc.mode == kGridSplitTail) tc = TileChoice{tc.cfg, inv::GRID_TILES, 1};
            // bytes a row sends up: fp32 X not normalised goes as bf16 operand rows
            const size_t x_up = (x_dtype == INV_DT_F32 && !nm) ? (size_t)W->ldw * 2
                                                               : (size_t)K * (x_dtype == INV_DT_F32 ? 4 : 2);
            const size_t up_row = x_up + (accumulate ? (size_t)N * ysz : 0);
            const int64_t mb = host_band_rows(tc, M, up_row, (size_t)N * ysz);
            if (mb > 0 && pipe_ready()) {
                BandExtras ex;
                ex.accumulate = accumulate;
                ex.gate = gd;
                if (nm) {
                    ex.nm = nm;
                    TRY(stage_norm_vectors(*nm, false, K, &ex.nscale, &ex.nshift));
                }
                return linear_host_banded(X, x_dtype, W, bd, Y, y_dtype, M, K, N, epilogue, tc, mb, ex);
            }
        }
        if (pipe_mode == 2)
            return fail(INV_ERR_UNSUPPORTED, "%s: INV_HIP_HOST_PIPELINE=2 but this call is not banded", who);
    }

    // Activations -> bf16 [M x ldw] (ldw = K rounded up to 8, zero padded), or
    // with INV_FLAG_PRECISE and fp32 X: [Xh | Xl], each half K rounded up to 64,
    // multiplied against the resident W read twice (the W k-tiles wrap).
    const uint16_t *Xd = nullptr;
    int64_t ldx = 0;
    const int64_t kseg = precise ? round_up(K, 64) : W->ldw;
    if (nm) {
        TRY(stage_normalized(who, (const float *)X, *nm, dev, M, K, &Xd, &ldx));
    } else {
        TRY(stage_operand(X, x_dtype, dev, false, M, K, K, precise ? 2 : 1, precise ? 0x2 : 0, precise ? 64 : 8,
                          g.x16, g.xin, &Xd, &ldx));
    }

    void *Yd = Y;
    if (!dev) {
        TRY(ensure(g.yout, (size_t)(M * N) * ysz));
        Yd = g.yout.p;
        if (accumulate) TRY(h2d_rows(Yd, Y, M, (size_t)N * ysz, (size_t)N * ysz));
    }
    // Accumulating reads Y as C (beta = 1) in place: every element is read and
    // then written by the one thread that finishes its tile.
    const float *cin = accumulate ? (const float *)Yd : nullptr;
    const float beta = accumulate ? 1.0f : 0.0f;
    // The GEMM runs over the handle's device rows (2 x 128-padded N for a
    // gate/up pair); Y has N columns either way.
    if (precise)
        TRY(run_gemm(W->w, W->ldw, Xd, ldx, Yd, N, out, bd, cin, N, 1.0f, beta, M, W->rows, 2 * kseg, epilogue,
                     kseg, W->ldw, N, gd));
    else
        TRY(run_gemm(W->w, W->ldw, Xd, ldx, Yd, N, out, bd, cin, N, 1.0f, beta, M, W->rows, W->ldw, epilogue,
                     0, -1, N, gd));
    g.calls++;
    if (!dev) {
        TRY(d2h_rows(Y, Yd, M, (size_t)N * ysz, (size_t)N * ysz));
    } else if (!(flags & INV_FLAG_ASYNC)) {
        HIPCHK(hipStreamSynchronize(g.stream));
    }
    return INV_OK;
}

// The library stream, its timing events and the two pinned bounce buffers.
int init_stream_objects() {
    HIPCHK(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
    for (hipEvent_t *e : {&g.tim0, &g.tim1, &g.st0, &g.st1}) HIPCHK(hipEventCreate(e));
    for (int k = 0; k < 2; ++k) {
        HIPCHK(hipEventCreateWithFlags(&g.pin_ev[k], hipEventDisableTiming));
        HIPCHK(hipEventRecord(g.pin_ev[k], g.stream));
        if (hipHostMalloc(&g.pin[k], kPinChunk, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            g.pin[k] = nullptr;
            return fail(INV_ERR_OOM, "pinned bounce buffer allocation failed");
        }
    }
    return INV_OK;
}

void release_stream_objects() {
    if (g.stream) (void)hipStreamSynchronize(g.stream);
    release_pipe();
    for (int k = 0; k < 2; ++k) {
        if (g.pin[k]) (void)hipHostFree(g.pin[k]);
        if (g.pin_ev[k]) (void)hipEventDestroy(g.pin_ev[k]);
        g.pin[k] = nullptr;
        g.pin_ev[k] = nullptr;
    }
    for (hipEvent_t *e : {&g.tim0, &g.tim1, &g.st0, &g.st1}) {
        if (*e) (void)hipEventDestroy(*e);
        *e = nullptr;
    }
    if (g.stream) (void)hipStreamDestroy(g.stream);
    g.stream = nullptr;
}

// x [rows x head_dim] fp32 (rows = tokens * heads): per-head RMSNorm (w, or
// none) then the rotary embedding (rope, tables ct/st), in place, or into y as
// bf16 when y is given.
int launch_head_norm_rope(float *x, uint16_t *y, int64_t rows, int64_t heads, int64_t head_dim, const float *w,
                          int rope, const float *ct, const float *st, int64_t ldx = 0) {
    if (rows == 0) return INV_OK;
    if (ldx == 0) ldx = heads * head_dim;
    const int64_t per_wg = 4 * inv::HNR_ROWS;
    if ((rows + per_wg - 1) / per_wg > INT32_MAX) return fail(INV_ERR_UNSUPPORTED, "head_norm_rope: too many rows");
    const dim3 grid((unsigned)((rows + per_wg - 1) / per_wg));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, g.stream, x, rows, (int)heads, w, ct, st, 1e-6f, y, ldx);
    };
    using namespace inv;
#define INV_HNR(EPT, OB)                                                                                  \
    do {                                                                                                  \
        if (!w) {                                                                                         \
            if (rope == INV_ROPE_INTERLEAVED) go(head_norm_rope<EPT, ROPE_INTERLEAVED, false, OB>);       \
            else if (rope == INV_ROPE_HALF) go(head_norm_rope<EPT, ROPE_HALF, false, OB>);                \
            else go(head_norm_rope<EPT, ROPE_NONE, false, OB>);                                           \
        } else if (rope == INV_ROPE_NONE) go(head_norm_rope<EPT, ROPE_NONE, true, OB>);                  \
        else if (rope == INV_ROPE_INTERLEAVED) go(head_norm_rope<EPT, ROPE_INTERLEAVED, true, OB>);      \
        else go(head_norm_rope<EPT, ROPE_HALF, true, OB>);                                                \
    } while (0)
    if (head_dim == 128) {
        if (y) INV_HNR(2, true);
        else INV_HNR(2, false);
    } else {
        if (y) INV_HNR(1, true);
        else INV_HNR(1, false);
    }
#undef INV_HNR
    HIPCHK(hipGetLastError());
    return INV_OK;
}

// The per-head RMSNorm and rotary embedding applied to Q and K while they are
// staged for attention (inv_hip_attention_qk_norm_rope).
struct QkPrep {
    const float *q_w, *k_w;  // RMSNorm weights [head_dim] or null
    int rope;                // INV_ROPE_*
    const float *q_cos, *q_sin, *k_cos, *k_sin;  // per-token tables or null
    int64_t ldq, ldk, ldv;   // token strides of Q, K, V in elements (packed: heads*head_dim)
};

// fp32 X [seq x nh*D] (host or device) -> norm + rotary -> bf16 [seq x nh*D] in dst.
// Host X, weight and tables are copied to the device first (vec: scratch for them).
int stage_prepped(const float *X, int64_t ldx, bool dev, int64_t seq, int64_t nh, int64_t D, const float *w, int rope,
                  const float *ct, const float *st, Buf &dst, Buf &tmp, Buf &vec, const uint16_t **out,
                  int64_t *out_ld) {
    const int64_t cols = nh * D;
    const int64_t width = (rope == INV_ROPE_HALF) ? D / 2 : D;
    const size_t xb = (size_t)(seq * cols) * 4, wb = (size_t)D * 4, tb = (size_t)(seq * width) * 4;
    const float *src = X;
    const float *wd = w, *cd = ct, *sd = st;
    if (!dev) {
        TRY(ensure(tmp, xb));
        TRY(h2d_rows(tmp.p, X, seq, (size_t)cols * 4, (size_t)ldx * 4));
        src = (const float *)tmp.p;
        ldx = cols;
        TRY(ensure(vec, wb + 2 * tb));
        char *vb = (char *)vec.p;
        if (w) TRY(h2d_rows(vb, w, 1, wb, wb));
        if (rope != INV_ROPE_NONE) {
            TRY(h2d_rows(vb + wb, ct, 1, tb, tb));
            TRY(h2d_rows(vb + wb + tb, st, 1, tb, tb));
        }
        wd = w ? (const float *)vb : nullptr;
        cd = (const float *)(vb + wb);
        sd = (const float *)(vb + wb + tb);
    } else if (!aligned(X, 8) || ldx % 2 || (w && !aligned(w, 4)) || (ct && !aligned(ct, 4)) || (st && !aligned(st, 4))) {
        return fail(INV_ERR_ARG, "attention: device Q/K must be 8-byte aligned with an even leading dimension, "
                                 "the norm/rotary vectors 4-byte aligned");
    }
    TRY(ensure(dst, (size_t)(seq * cols) * 2));
    TRY(launch_head_norm_rope(const_cast<float *>(src), (uint16_t *)dst.p, seq * nh, nh, D, wd, rope, cd, sd, ldx));
    *out = (const uint16_t *)dst.p;
    *out_ld = cols;
    return INV_OK;
}

// Query-key pairs an attention call evaluates: all of them, or (causal) key j
// <= i + offset for query i, offset = seq_k - seq_q.
double attention_pairs(int64_t sq, int64_t sk, bool causal) {
    if (!causal) return (double)sq * (double)sk;
    double n = 0.0;
    const int64_t off = sk - sq;
    // query i sees clamp(i + off + 1, 0, sk) keys: zero below i0, sk from i1 on
    const int64_t i0 = std::min<int64_t>(sq, std::max<int64_t>(0, -off));
    const int64_t i1 = std::min<int64_t>(sq, std::max<int64_t>(i0, sk - off - 1));
    // i in [i0, i1): i + off + 1 keys, an arithmetic series
    n += (double)(i1 - i0) * (double)(i0 + i1 - 1) / 2.0 + (double)(i1 - i0) * (double)(off + 1);
    n += (double)(sq - i1) * (double)sk;
    return n;
}

int attention_impl(const void *Q, const void *K, const void *V, void *O, int in_dtype, int out_dtype, int64_t heads,
                   int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim, float scale,
                   const int32_t *key_mask, int flags, const QkPrep *prep = nullptr) {
    TRY(check_init());
    if (in_dtype != INV_DT_F32 && in_dtype != INV_DT_BF16) return fail(INV_ERR_ARG, "attention: bad in_dtype %d", in_dtype);
    if (out_dtype != INV_DT_F32 && out_dtype != INV_DT_BF16)
        return fail(INV_ERR_ARG, "attention: bad out_dtype %d", out_dtype);
    if (flags & ~(INV_FLAG_DEVICE_PTRS | INV_FLAG_ASYNC | INV_ATTN_CAUSAL))
        return fail(INV_ERR_ARG, "attention: unknown flags 0x%x", flags);
    if ((flags & INV_FLAG_ASYNC) && !(flags & INV_FLAG_DEVICE_PTRS))
        return fail(INV_ERR_ARG, "attention: ASYNC requires DEVICE_PTRS");
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
        return fail(INV_ERR_ARG, "attention: heads (%lld) must be a positive multiple of kv_heads (%lld)",
                    (long long)heads, (long long)kv_heads);
    if (seq_q < 0 || seq_k < 0) return fail(INV_ERR_ARG, "attention: negative sequence length");
    if (head_dim != 64 && head_dim != 128)
        return fail(INV_ERR_UNSUPPORTED, "attention: head_dim %lld (64 and 128 are supported)", (long long)head_dim);
    if (!(scale > 0.0f) || scale > 3.0e38f) return fail(INV_ERR_ARG, "attention: scale must be positive and finite");
    if (seq_q == 0) return INV_OK;
    if (seq_k == 0) return fail(INV_ERR_ARG, "attention: seq_k is 0 (a softmax over no keys)");
    if (!Q || !K || !V || !O) return fail(INV_ERR_ARG, "attention: Q, K, V or O is null");
    if (seq_q > INT32_MAX / 2 || seq_k > INT32_MAX / 2 ||
        ((seq_q + 63) / 64) * heads > INT32_MAX)
        return fail(INV_ERR_UNSUPPORTED, "attention: too many heads or tokens");
    const int64_t hq = heads * head_dim, hk = kv_heads * head_dim;
    // K and V are staged with leading dimension round_up(hk, 8) (or used in place at hk)
    if (seq_k * round_up(hk, 8) * 2 >= ((int64_t)1 << 31))
        return fail(INV_ERR_UNSUPPORTED, "attention: K or V above 2 GiB (32-bit buffer offsets)");
    const bool dev = (flags & INV_FLAG_DEVICE_PTRS) != 0;
    const size_t osz = out_dtype == INV_DT_F32 ? 4 : 2;
    if (dev && !aligned(O, 16)) return fail(INV_ERR_ARG, "attention: device O must be 16-byte aligned");
    if (dev && key_mask && !aligned(key_mask, 4)) return fail(INV_ERR_ARG, "attention: device key_mask not 4-byte aligned");

    const bool causal = (flags & INV_ATTN_CAUSAL) != 0;
    // Two key groups (64-query workgroups) where the 128-query grid leaves CUs
    // idle: Qwen3's 512-token prefill is 128 blocks on 256 CUs.
    // INV_HIP_ATTN_KEY_GROUPS=1 or 2 forces the choice.
    const int64_t blocks128 = ((seq_q + inv::kAttnBlockQ - 1) / inv::kAttnBlockQ) * heads;
    int key_groups = blocks128 < (g.cu_count > 0 ? g.cu_count : 256) ? 2 : 1;
    const int kg_ov = env_int("INV_HIP_ATTN_KEY_GROUPS", 0);
    if (kg_ov == 1 || kg_ov == 2) key_groups = kg_ov;
    // Host Q and O: query-row bands through the band pipeline (K and V first,
    // whole); bands are whole query blocks of the whole problem's workgroup
    // shape, so each query's result is the one-launch result.
    const int64_t band_q =
        (!dev && !prep && !g.stats && env_int("INV_HIP_HOST_PIPELINE", 1))
            ? host_band_rows(inv::kAttnBlockQ / key_groups, seq_q, (size_t)hq * 2, (size_t)hq * osz) : 0;
    const bool banded = band_q > 0 && pipe_ready();
    if (!dev && !banded && env_int("INV_HIP_HOST_PIPELINE", 1) == 2)
        return fail(INV_ERR_UNSUPPORTED, "attention: INV_HIP_HOST_PIPELINE=2 but this call is not banded");

    // bf16 operands: Q, K and V row-major as given (in place when already bf16
    // on the device); the kernel reads V^T fragments with transposing LDS reads.
    const uint16_t *Qd = nullptr, *Kd = nullptr, *Vd = nullptr;
    int64_t ldq = 0, ldk = 0, ldv = 0;
    if (prep) {
        if (in_dtype != INV_DT_F32) return fail(INV_ERR_ARG, "attention: the Q/K norm and rotary need fp32 Q and K");
        if (prep->rope != INV_ROPE_NONE && prep->rope != INV_ROPE_INTERLEAVED && prep->rope != INV_ROPE_HALF)
            return fail(INV_ERR_ARG, "attention: bad rope mode %d", prep->rope);
        if (prep->rope != INV_ROPE_NONE && (!prep->q_cos || !prep->q_sin || !prep->k_cos || !prep->k_sin))
            return fail(INV_ERR_ARG, "attention: rotary tables are null");
        TRY(stage_prepped((const float *)Q, prep->ldq, dev, seq_q, heads, head_dim, prep->q_w, prep->rope,
                          prep->q_cos, prep->q_sin, g.aq, g.aqin, g.hvec, &Qd, &ldq));
        TRY(stage_prepped((const float *)K, prep->ldk, dev, seq_k, kv_heads, head_dim, prep->k_w, prep->rope,
                          prep->k_cos, prep->k_sin, g.ak, g.akin, g.hx, &Kd, &ldk));
    } else {
        if (!banded) TRY(stage_operand(Q, in_dtype, dev, false, seq_q, hq, hq, 1, 0, 8, g.aq, g.aqin, &Qd, &ldq));
        TRY(stage_operand(K, in_dtype, dev, false, seq_k, hk, hk, 1, 0, 8, g.ak, g.akin, &Kd, &ldk));
    }
    TRY(stage_operand(V, in_dtype, dev, false, seq_k, hk, prep ? prep->ldv : hk, 1, 0, 8, g.avt, g.avin, &Vd, &ldv));
    void *Od = O;
    if (!dev) {
        TRY(ensure(g.yout, (size_t)(seq_q * hq) * osz));
        Od = g.yout.p;
    }
    inv::AttnParams p{};
    p.Q = Qd;
    p.K = Kd;
    p.V = Vd;
    p.O = Od;
    p.ldq = ldq;
    p.ldk = ldk;
    p.ldv = ldv;
    p.ldo = hq;
    p.seq_q = (int)seq_q;
    p.seq_k = (int)seq_k;
    p.heads = (int)heads;
    p.kv_heads = (int)kv_heads;
    p.scale_log2 = scale * 1.44269504088896341f;
    p.causal_offset = (int)(seq_k - seq_q);
    p.key_mask = key_mask;
    if (key_mask && !dev) {
        TRY(ensure(g.amask, (size_t)seq_k * 4));
        TRY(h2d_rows(g.amask.p, key_mask, 1, (size_t)seq_k * 4, (size_t)seq_k * 4));
        p.key_mask = (const int32_t *)g.amask.p;
    }
    if (banded) {
        // a band's host Q rows go up as bf16 operand rows (fp32 rounded by the
        // host on the way into the bounce buffer), and its queries run as a
        // smaller problem whose causal offset counts from the band's first row
        const size_t row16 = (size_t)hq * 2, out_row = (size_t)hq * osz;
        TRY(ensure(g.aq, (size_t)seq_q * row16));
        auto stage = [&](int64_t r0, int64_t nr, char *pin) -> int {
            if (in_dtype == INV_DT_F32)
                par_cvt_rows((uint16_t *)pin, hq, (const float *)Q + r0 * hq, hq, nr, hq, hq);
            else
                par_copy_rows(pin, row16, (const char *)Q + r0 * row16, row16, nr, row16);
            HIPCHK(hipMemcpyAsync((char *)g.aq.p + (size_t)r0 * row16, pin, (size_t)nr * row16, hipMemcpyHostToDevice,
                                  g.pipe.up));
            return INV_OK;
        };
        auto compute = [&](int64_t r0, int64_t nr) -> int {
            uint16_t *qb = (uint16_t *)g.aq.p + r0 * hq;
            inv::AttnParams pb = p;
            pb.Q = qb;
            pb.ldq = hq;
            pb.seq_q = (int)nr;
            pb.O = (char *)g.yout.p + (size_t)r0 * out_row;
            pb.causal_offset = p.causal_offset + (int)r0;
            HIPCHK(inv::attention_launch(pb, (int)head_dim, causal, out_dtype == INV_DT_BF16 ? 1 : 0, key_groups,
                                         g.stream));
            return INV_OK;
        };
        TRY(run_band_pipeline(seq_q, band_q, (char *)O, out_row, (const char *)g.yout.p, stage, compute));
        g.calls++;
        return INV_OK;
    }
    if (g.stats) HIPCHK(hipEventRecord(g.st0, g.stream));
    HIPCHK(inv::attention_launch(p, (int)head_dim, causal, out_dtype == INV_DT_BF16 ? 1 : 0, key_groups, g.stream));
    if (g.stats) {
        HIPCHK(hipEventRecord(g.st1, g.stream));
        HIPCHK(hipEventSynchronize(g.st1));
        float ms = 0.f;
        HIPCHK(hipEventElapsedTime(&ms, g.st0, g.st1));
        g.gemm_ms += ms;
        g.flops += 4.0 * attention_pairs(seq_q, seq_k, causal) * (double)head_dim * (double)heads;
    }
    g.calls++;
    if (!dev) {
        TRY(d2h_rows(O, Od, seq_q, (size_t)hq * osz, (size_t)hq * osz));
    } else if (!(flags & INV_FLAG_ASYNC)) {
        HIPCHK(hipStreamSynchronize(g.stream));
    }
    return INV_OK;
}

// Per-head RMSNorm and rotary embedding of Q or K in place (fp32).
// Convolution as a GEMM per image (QNNConv2d, src/quicknncpu.pas:1958-2124):
// Y[oc][p] = sum_k Wt[oc][k] * col[p][k] + bias[oc], with the patch matrix col
// built by im2col_bf16 (pixel-major, K contiguous) and the weights as the
// GEMM's X operand, so the output lands in NCHW order with the bias added per
// row.  Output rows are taken in chunks whose patch matrix fits kColCap bytes
// (INV_HIP_CONV_COL_MB overrides it, in MiB).
constexpr size_t kColCap = (size_t)1 << 30;

// Tile configuration of the implicit convolution, or -1 for the patch-matrix
// path: in_ch a multiple of 64 (a k-tile is 64 channels of one tap), at most
// 31 taps (one mask bit each), an NHWC bf16 image below 2 GiB (32-bit buffer
// offsets), at least 64 output channels, more than one tap and half a round
// of tiles.  256x128
// tiles (configuration 13) for up to 128 output channels, else 256x256 (9,
// one register stage) or 256x224 (16), as the plain GEMM would choose between
// its 256x256 and 256x224 tiles.  INV_HIP_CONV_GATHER=0 turns it off, =2
// takes it whatever the tile count (where it applies at all).
int conv_gather_cfg(int64_t in_ch, int64_t out_ch, int64_t H, int64_t W, int64_t taps, int64_t P) {
    const int mode = env_int("INV_HIP_CONV_GATHER", 1);
    // 1x1: the patch matrix is the image transposed, the same bytes as the
    // NHWC copy, and the plain GEMM measured faster (0.54 against 0.58 ms at
    // 1024x1024, 256 -> 128)
    if (!mode || (taps == 1 && mode != 2)) return -1;
    if (in_ch % 64 || taps > 31 || out_ch < 64 || H * W * in_ch * 2 >= ((int64_t)1 << 31)) return -1;
    if (P > INT32_MAX / 2 || out_ch * in_ch * taps > ((int64_t)1 << 31)) return -1;
    const int cus = g.cu_count > 0 ? g.cu_count : 256;
    int cfg = 13;
    if (out_ch > 128) {
        // the GEMM's own choice where it has a gather loader (16, 13), else the
        // 4-wave 256x256 tile (the 8-wave one gathers slower: 450 against 314 us
        // at 512 channels x 256^2); 13 keeps 512 channels x 128^2 at one full
        // round of 256 tiles (95 us, against 120 for 128 tiles of 256x256)
        const TileChoice tc = choose_tiles(out_ch, P, in_ch * taps);
        cfg = (tc.cfg == 16 || tc.cfg == 13) ? tc.cfg : 9;
    }
    const int ov = env_int("INV_HIP_CONV_GATHER_CFG", -1);
    if (ov == 9 || ov == 13 || ov == 16) cfg = ov;
    const int64_t tiles = ((out_ch + kCfg[cfg].tm - 1) / kCfg[cfg].tm) * ((P + kCfg[cfg].tn - 1) / kCfg[cfg].tn);
    return (mode == 2 || tiles * 2 >= cus) ? cfg : -1;
}

// The direct 3x3 kernel for at most 8 output channels on an fp32 or bf16 image.
template <typename T>
int launch_conv3x3_thin(dim3 grid, const T *sd, inv_weight_t Wt, const float *bd, float *yd, int64_t in_ch, int64_t H,
                        int64_t W, int64_t padding, int64_t out_ch, int64_t outH, int64_t outW) {
    if (out_ch <= 3)  // RGB
        hipLaunchKernelGGL((inv::conv3x3_thin<3, T>), grid, dim3(256), 0, g.stream, sd, Wt->w, Wt->ldw, bd, yd,
                           (int)in_ch, (int)H, (int)W, (int)padding, (int)out_ch, (int)outH, (int)outW);
    else if (out_ch <= 4)
        hipLaunchKernelGGL((inv::conv3x3_thin<4, T>), grid, dim3(256), 0, g.stream, sd, Wt->w, Wt->ldw, bd, yd,
                           (int)in_ch, (int)H, (int)W, (int)padding, (int)out_ch, (int)outH, (int)outW);
    else
        hipLaunchKernelGGL((inv::conv3x3_thin<8, T>), grid, dim3(256), 0, g.stream, sd, Wt->w, Wt->ldw, bd, yd,
                           (int)in_ch, (int)H, (int)W, (int)padding, (int)out_ch, (int)outH, (int)outW);
    HIPCHK(hipGetLastError());
    return INV_OK;
}

int conv2d_impl(const float *src, inv_weight_t Wt, const float *bias, float *dst, int64_t in_ch, int64_t out_ch,
                int64_t H, int64_t W, int64_t kH, int64_t kW, int64_t stride, int64_t padding, int64_t batch,
                int flags) {
    TRY(check_init());
    if (!valid_weight(Wt)) return fail(INV_ERR_ARG, "conv2d: unknown weight handle");
    if (flags & ~(INV_FLAG_DEVICE_PTRS | INV_FLAG_ASYNC)) return fail(INV_ERR_ARG, "conv2d: unknown flags 0x%x", flags);
    if ((flags & INV_FLAG_ASYNC) && !(flags & INV_FLAG_DEVICE_PTRS))
        return fail(INV_ERR_ARG, "conv2d: ASYNC requires DEVICE_PTRS");
    if (in_ch <= 0 || out_ch <= 0 || H <= 0 || W <= 0 || kH <= 0 || kW <= 0 || stride <= 0 || padding < 0 || batch < 0)
        return fail(INV_ERR_ARG, "conv2d: bad shape");
    const int64_t outH = (H + 2 * padding - kH) / stride + 1, outW = (W + 2 * padding - kW) / stride + 1;
    if (H + 2 * padding < kH || W + 2 * padding < kW) return fail(INV_ERR_ARG, "conv2d: kernel larger than the padded image");
    const int64_t K = in_ch * kH * kW;
    if (Wt->gated || Wt->N != out_ch || Wt->K != K)
        return fail(INV_ERR_ARG, "conv2d: weight is %lld x %lld, the call needs %lld x %lld (out_ch x in_ch*kH*kW)",
                    (long long)Wt->N, (long long)Wt->K, (long long)out_ch, (long long)K);
    const int64_t P = outH * outW, img = in_ch * H * W;
    if (H > INT32_MAX / 4 || W > INT32_MAX / 4 || kH > 65536 || kW > 65536 || stride > INT32_MAX / 4 ||
        padding > INT32_MAX / 4 || K > ((int64_t)1 << 21) || img > ((int64_t)1 << 40) || P > INT32_MAX / 2)
        return fail(INV_ERR_UNSUPPORTED, "conv2d: dimensions too large");
    if (batch == 0) return INV_OK;
    if (!src || !dst) return fail(INV_ERR_ARG, "conv2d: src or dst is null");
    const bool dev = (flags & INV_FLAG_DEVICE_PTRS) != 0;
    const int64_t ldc = round_up(K, 64);  // patch-matrix row pitch: whole 128-byte segments

    // Bias: explicit argument first, else the handle's.
    const float *bd = Wt->bias;
    if (bias) {
        if (dev && aligned(bias, 4)) {
            bd = bias;
        } else {
            TRY(ensure(g.bias, (size_t)out_ch * 4));
            if (dev)
                HIPCHK(hipMemcpyAsync(g.bias.p, bias, (size_t)out_ch * 4, hipMemcpyDeviceToDevice, g.stream));
            else
                TRY(h2d_rows(g.bias.p, bias, 1, (size_t)out_ch * 4, (size_t)out_ch * 4));
            bd = (const float *)g.bias.p;
        }
    }
    // A host image goes up rounded to bf16 by the host (every path rounds it
    // to bf16 before use, so the results are the bits of an fp32 upload): sd16.
    const float *sd = src;
    const uint16_t *sd16 = nullptr;
    float *yd = dst;
    const size_t sbytes = (size_t)(batch * img) * 4, ybytes = (size_t)(batch * out_ch * P) * 4;
    if (!dev) {
        if ((size_t)W * 2 <= kPinChunk) {
            TRY(ensure(g.csrc, sbytes / 2));
            TRY(h2d_rows_bf16((uint16_t *)g.csrc.p, src, batch * in_ch * H, W, W, W));
            sd16 = (const uint16_t *)g.csrc.p;
            sd = nullptr;
        } else {
            TRY(ensure(g.csrc, sbytes));
            TRY(h2d_rows(g.csrc.p, src, 1, sbytes, sbytes));
            sd = (const float *)g.csrc.p;
        }
        TRY(ensure(g.cdst, ybytes));
        yd = (float *)g.cdst.p;
    } else if (!aligned(src, 4) || !aligned(dst, 4)) {
        return fail(INV_ERR_ARG, "conv2d: src and dst must be 4-byte aligned");
    }
    // Few output channels, 3x3 at stride 1 (conv_out): the direct kernel, no patch matrix.
    if (kH == 3 && kW == 3 && stride == 1 && out_ch <= 8 && batch <= 65535 && env_int("INV_HIP_CONV_DIRECT", 1)) {
        const dim3 grid((unsigned)((outW + inv::CT_TW - 1) / inv::CT_TW), (unsigned)((outH + inv::CT_TH - 1) / inv::CT_TH),
                        (unsigned)batch);
        if (grid.y > 65535) return fail(INV_ERR_UNSUPPORTED, "conv2d: image too tall");
        if ((int64_t)grid.x * grid.y * grid.z > INT32_MAX) return fail(INV_ERR_UNSUPPORTED, "conv2d: too many tiles");
        if (sd16)
            TRY(launch_conv3x3_thin(grid, sd16, Wt, bd, yd, in_ch, H, W, padding, out_ch, outH, outW));
        else
            TRY(launch_conv3x3_thin(grid, sd, Wt, bd, yd, in_ch, H, W, padding, out_ch, outH, outW));
        g.calls++;
        if (!dev) {
            TRY(d2h_rows(dst, yd, 1, ybytes, ybytes));
        } else if (!(flags & INV_FLAG_ASYNC)) {
            HIPCHK(hipStreamSynchronize(g.stream));
        }
        return INV_OK;
    }
    // Many channels in and out: the implicit GEMM, whose loader gathers each
    // k-tile (64 channels of one tap) straight from an NHWC bf16 copy of the
    // image, so no patch matrix is written or read.
    const int gcfg = conv_gather_cfg(in_ch, out_ch, H, W, kH * kW, P);
    if (gcfg >= 0) {
        const int64_t taps = kH * kW, HW = H * W;
        TRY(ensure(g.cimg, (size_t)(HW * in_ch) * 2));
        TRY(ensure(g.cfilt, (size_t)(out_ch * K) * 2));
        uint16_t *nhwc = (uint16_t *)g.cimg.p, *filt = (uint16_t *)g.cfilt.p;
        const int64_t total = out_ch * K;
        hipLaunchKernelGGL(inv::conv_filter_tap_major, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g.stream,
                           Wt->w, Wt->ldw, filt, (int)in_ch, (int)taps, total);
        HIPCHK(hipGetLastError());
        if (!bd) {  // the per-row bias epilogue always adds one
            TRY(ensure(g.bias, (size_t)out_ch * 4));
            hipLaunchKernelGGL(fill_zero_u32, dim3((unsigned)((out_ch + 255) / 256)), dim3(256), 0, g.stream,
                               (unsigned *)g.bias.p, out_ch);
            HIPCHK(hipGetLastError());
            bd = (const float *)g.bias.p;
        }
        const CfgMeta &cm = kCfg[gcfg];
        inv::GemmParams p{};
        p.X = filt;
        p.ldx = K;
        p.ldy = P;
        p.M = (int)out_ch;
        p.N = (int)P;
        p.K = (int)K;
        p.Kw = (int)K;
        p.tiles_m = (int)((out_ch + cm.tm - 1) / cm.tm);
        p.tiles_n = (int)((P + cm.tn - 1) / cm.tn);
        p.group_m = std::max(1, std::min(p.tiles_m, env_int("INV_HIP_GROUP_M", 8)));
        p.alpha = 1.0f;
        p.row_bias = bd;
        p.ksplit = 1;
        p.kt_per_split = (int)(K / 64);
        p.cv_H = (int)H;
        p.cv_W = (int)W;
        p.cv_C = (int)in_ch;
        p.cv_outW = (int)outW;
        p.cv_kW = (int)kW;
        p.cv_taps = (int)taps;
        p.cv_stride = (int)stride;
        p.cv_pad = (int)padding;
        for (int64_t b = 0; b < batch; ++b) {
            // image b: [C x HW] fp32 (or bf16) -> [HW x C] bf16
            if (sd16)
                TRY(launch_transpose<uint16_t>(sd16 + b * img, HW, nhwc, in_ch, in_ch, HW, in_ch));
            else
                TRY(launch_transpose<float>(sd + b * img, HW, nhwc, in_ch, in_ch, HW, in_ch));
            p.W = nhwc;
            p.Y = yd + b * out_ch * P;
            p.vec_store = (P % 4 == 0) && aligned(p.Y, 16);
            if (g.stats) HIPCHK(hipEventRecord(g.st0, g.stream));
            HIPCHK(cm.launch(p, inv::EPI_ROWBIAS, inv::OUT_F32, inv::LAUNCH_GATHER, g.stream));
            if (g.stats) {
                HIPCHK(hipEventRecord(g.st1, g.stream));
                HIPCHK(hipEventSynchronize(g.st1));
                float ms = 0.f;
                HIPCHK(hipEventElapsedTime(&ms, g.st0, g.st1));
                g.gemm_ms += ms;
                g.flops += 2.0 * (double)out_ch * (double)P * (double)K;
            }
        }
        g.calls++;
        if (!dev) {
            TRY(d2h_rows(dst, yd, 1, ybytes, ybytes));
        } else if (!(flags & INV_FLAG_ASYNC)) {
            HIPCHK(hipStreamSynchronize(g.stream));
        }
        return INV_OK;
    }
    const int64_t row_bytes = outW * ldc * 2;
    const int64_t cap = std::max(1, env_int("INV_HIP_CONV_COL_MB", (int)(kColCap >> 20))) * ((int64_t)1 << 20);
    const int64_t chunk_rows = std::max<int64_t>(1, std::min<int64_t>(outH, cap / row_bytes));
    TRY(ensure(g.ccol, (size_t)(chunk_rows * row_bytes)));
    uint16_t *col = (uint16_t *)g.ccol.p;
    for (int64_t b = 0; b < batch; ++b) {
        float *out_b = yd + b * out_ch * P;
        for (int64_t oh0 = 0; oh0 < outH; oh0 += chunk_rows) {
            const int64_t rows = std::min(chunk_rows, outH - oh0), npix = rows * outW;
            const dim3 grid((unsigned)((npix + 64 * inv::IM2COL_PG - 1) / (64 * inv::IM2COL_PG)), (unsigned)(ldc / 64));
            if (sd16)
                hipLaunchKernelGGL(inv::im2col_bf16<uint16_t>, grid, dim3(512), 0, g.stream, sd16 + b * img, col,
                                   (int)H, (int)W, (int)kH, (int)kW, (int)stride, (int)padding, (int)outW, (int)oh0,
                                   npix, (int)K, ldc);
            else
                hipLaunchKernelGGL(inv::im2col_bf16<float>, grid, dim3(512), 0, g.stream, sd + b * img, col, (int)H,
                                   (int)W, (int)kH, (int)kW, (int)stride, (int)padding, (int)outW, (int)oh0, npix,
                                   (int)K, ldc);
            HIPCHK(hipGetLastError());
            // Y[oc][oh0*outW + q] (row pitch P) = Wt[oc] . col[q] + bias[oc]
            TRY(run_gemm(col, ldc, Wt->w, Wt->ldw, out_b + oh0 * outW, P, inv::OUT_F32, nullptr, nullptr, 0, 1.0f,
                         0.0f, out_ch, npix, Wt->ldw, INV_EPI_NONE, 0, -1, -1, nullptr, bd));
        }
    }
    g.calls++;
    if (!dev) {
        TRY(d2h_rows(dst, yd, 1, ybytes, ybytes));
    } else if (!(flags & INV_FLAG_ASYNC)) {
        HIPCHK(hipStreamSynchronize(g.stream));
    }
    return INV_OK;
}

int head_norm_rope_impl(float *X, int64_t seq, int64_t heads, int64_t head_dim, const float *w, int rope,
                        const float *ct, const float *st, int flags) {
    TRY(check_init());
    if (flags & ~(INV_FLAG_DEVICE_PTRS | INV_FLAG_ASYNC)) return fail(INV_ERR_ARG, "head_norm_rope: unknown flags 0x%x", flags);
    if ((flags & INV_FLAG_ASYNC) && !(flags & INV_FLAG_DEVICE_PTRS))
        return fail(INV_ERR_ARG, "head_norm_rope: ASYNC requires DEVICE_PTRS");
    if (seq < 0 || heads <= 0) return fail(INV_ERR_ARG, "head_norm_rope: bad shape");
    if (head_dim != 64 && head_dim != 128)
        return fail(INV_ERR_UNSUPPORTED, "head_norm_rope: head_dim %lld (64 and 128 are supported)", (long long)head_dim);
    if (rope != INV_ROPE_NONE && rope != INV_ROPE_INTERLEAVED && rope != INV_ROPE_HALF)
        return fail(INV_ERR_ARG, "head_norm_rope: bad rope mode %d", rope);
    if (rope != INV_ROPE_NONE && (!ct || !st)) return fail(INV_ERR_ARG, "head_norm_rope: rotary tables are null");
    if (seq == 0 || (!w && rope == INV_ROPE_NONE)) return INV_OK;
    if (!X) return fail(INV_ERR_ARG, "head_norm_rope: X is null");
    const int64_t rows = seq * heads;
    if (rows > ((int64_t)1 << 33)) return fail(INV_ERR_UNSUPPORTED, "head_norm_rope: too many rows");
    const bool dev = (flags & INV_FLAG_DEVICE_PTRS) != 0;
    const int64_t width = (rope == INV_ROPE_HALF) ? head_dim / 2 : head_dim;  // table columns per token
    const size_t xb = (size_t)(rows * head_dim) * 4, tb = (size_t)(seq * width) * 4, wb = (size_t)head_dim * 4;
    float *xd = X;
    const float *wd = w, *cd = ct, *sd = st;
    if (!dev) {
        TRY(ensure(g.hx, xb));
        TRY(h2d_rows(g.hx.p, X, 1, xb, xb));
        xd = (float *)g.hx.p;
        TRY(ensure(g.hvec, wb + 2 * tb));
        char *vb = (char *)g.hvec.p;
        if (w) TRY(h2d_rows(vb, w, 1, wb, wb));
        if (rope != INV_ROPE_NONE) {
            TRY(h2d_rows(vb + wb, ct, 1, tb, tb));
            TRY(h2d_rows(vb + wb + tb, st, 1, tb, tb));
        }
        wd = w ? (const float *)vb : nullptr;
        cd = (const float *)(vb + wb);
        sd = (const float *)(vb + wb + tb);
    } else if (!aligned(X, 8) || (w && !aligned(w, 4)) || (ct && !aligned(ct, 4)) || (st && !aligned(st, 4))) {
        return fail(INV_ERR_ARG, "head_norm_rope: X must be 8-byte and the vectors 4-byte aligned");
    }
    TRY(launch_head_norm_rope(xd, nullptr, rows, heads, head_dim, wd, rope, cd, sd));
    if (!dev) {
        TRY(d2h_rows(X, xd, 1, xb, xb));
    } else if (!(flags & INV_FLAG_ASYNC)) {
        HIPCHK(hipStreamSynchronize(g.stream));
    }
    return INV_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" {

int inv_hip_abi_version(void) { return INV_HIP_ABI_VERSION; }

const char *inv_hip_last_error(void) { return t_err.c_str(); }

int inv_hip_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g.init) {
        if (device == g.device) return INV_OK;
        return fail(INV_ERR_ARG, "already initialised on device %d", g.device);
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return fail(INV_ERR_NO_DEVICE, "no HIP device visible");
    }
    if (device < 0 || device >= n) return fail(INV_ERR_NO_DEVICE, "device %d out of range (%d visible)", device, n);
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(INV_ERR_NO_DEVICE, "device %d is %s, this library is built for gfx950", device, prop.gcnArchName);
    HIPCHK(hipSetDevice(device));
    const int rc = init_stream_objects();
    if (rc) {
        release_stream_objects();  // a later call may try again from scratch
        return rc;
    }
    // The device address of this GPU's scratch array (the array's name is a
    // host-side stand-in, never an address).
    void *sp = nullptr;
    const hipError_t se = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (se != hipSuccess || !sp) {
        (void)hipGetLastError();
        release_stream_objects();
        return fail(INV_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(se));
    }
    g.scratch = (unsigned char *)sp;
    g.device = device;
    g.cu_count = prop.multiProcessorCount;
    g.clock_khz = prop.clockRate;
    g.alloc_cap = (size_t)std::max(0, env_int("INV_HIP_ALLOC_LIMIT_MB", 0)) << 20;
    g.alloc_base = g.alloc_bytes;
    // the product name when the runtime reports one, else the architecture and CU count
    char pname[256] = {0};
    if (hipDeviceGetName(pname, sizeof pname, device) != hipSuccess) (void)hipGetLastError();
    const char *nm = pname[0] ? pname : prop.name;
    if (nm[0])
        snprintf(g.name, sizeof g.name, "%s (%s)", nm, prop.gcnArchName);
    else
        snprintf(g.name, sizeof g.name, "AMD GPU %s, %d CUs", prop.gcnArchName, prop.multiProcessorCount);
    // host copy threads: INV_HIP_COPY_THREADS, else up to 8 of the host's
    const char *ct = getenv("INV_HIP_COPY_THREADS");
    const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
    g_copy.start(std::max(1, std::min(64, (ct && *ct) ? atoi(ct) : std::min(8, hw))));
    g.init = true;
    return INV_OK;
}

int inv_hip_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g.init) return INV_OK;
    (void)hipSetDevice(g.device);
    (void)hipStreamSynchronize(g.stream);
    for (auto *w : g.weights) free_weight(w);
    g.weights.clear();
    g.cache.clear();
    g.cache_bytes = 0;
    g.cache_budget = 0;
    g.cache_clock = 0;
    g.cache_hits = g.cache_misses = g.cache_uploaded = 0;
    for (Buf *b : {&g.xin, &g.x16, &g.w16, &g.win, &g.yout, &g.cin, &g.bias, &g.gate, &g.aq, &g.ak, &g.avt, &g.aqin,
                   &g.akin, &g.avin, &g.nvec, &g.amask, &g.hx, &g.hvec, &g.csrc, &g.ccol, &g.cdst, &g.cimg, &g.cfilt})
        release(*b);
    // g.partial / g.counters (uncached) stay allocated until the process ends.
    release_stream_objects();
    g_copy.stop_all();
    g.init = false;
    g.scratch = nullptr;
    g.device = -1;
    g.stats = false;
    g.calls = 0;
    g.gemm_ms = g.flops = 0.0;
    return INV_OK;
}

int inv_hip_device_info(char *name, size_t name_len, int *cu_count, int *clock_khz) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (name && name_len) snprintf(name, name_len, "%s", g.name);
    if (cu_count) *cu_count = g.cu_count;
    if (clock_khz) *clock_khz = g.clock_khz;
    return INV_OK;
}

int inv_hip_weight_upload(const uint16_t *w_bf16, int64_t N, int64_t K, const float *bias, inv_weight_t *out) {
    std::lock_guard<std::mutex> lk(g_mu);
    return weight_upload_impl(w_bf16, false, N, K, bias, out);
}

int inv_hip_weight_upload_f32(const float *w_f32, int64_t N, int64_t K, const float *bias, inv_weight_t *out) {
    std::lock_guard<std::mutex> lk(g_mu);
    return weight_upload_impl(w_f32, true, N, K, bias, out);
}

int inv_hip_weight_upload_gate_up(const uint16_t *gate_bf16, const uint16_t *up_bf16, int64_t F, int64_t K,
                                  const float *gate_bias, const float *up_bias, inv_weight_t *out) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!out) return fail(INV_ERR_ARG, "out handle pointer is null");
    *out = nullptr;
    if (!gate_bf16 || !up_bf16 || F <= 0 || K <= 0)
        return fail(INV_ERR_ARG, "gate/up weight: null pointer or non-positive shape (F=%lld K=%lld)", (long long)F,
                    (long long)K);
    if (F > INT32_MAX / 8 || K > INT32_MAX / 2) return fail(INV_ERR_ARG, "gate/up weight too large");
    const int64_t ldw = round_up(K, 8), fpad = round_up(F, 128), rows = 2 * fpad;
    uint16_t *dw = nullptr;
    TRY(dev_alloc((void **)&dw, (size_t)(rows * ldw) * 2, "gate/up weight"));
    int rc = INV_OK;
    if (hipMemsetAsync(dw, 0, (size_t)(rows * ldw) * 2, g.stream) != hipSuccess)
        rc = fail(INV_ERR_HIP, "gate/up weight: clearing failed");
    // 128-row blocks: gate rows [128b, 128b+128) -> device rows 256b.., up -> 256b+128..
    for (int half = 0; half < 2 && !rc; ++half) {
        const uint16_t *src = half ? up_bf16 : gate_bf16;
        for (int64_t f0 = 0; f0 < F && !rc; f0 += 128) {
            const int64_t nr = std::min<int64_t>(128, F - f0);
            uint16_t *dst = dw + ((f0 / 128) * 256 + half * 128) * ldw;
            if (ldw == K) {
                rc = h2d_rows(dst, src + f0 * K, nr, (size_t)K * 2, (size_t)K * 2);
            } else {
                rc = ensure(g.win, (size_t)(nr * K) * 2);
                if (!rc) rc = h2d_rows(g.win.p, src + f0 * K, nr, (size_t)K * 2, (size_t)K * 2);
                if (!rc) rc = launch_copy_rows_bf16((const uint16_t *)g.win.p, K, dst, ldw, nr, K, ldw);
                if (!rc && hipStreamSynchronize(g.stream) != hipSuccess) rc = fail(INV_ERR_HIP, "gate/up copy failed");
            }
        }
    }
    float *db = nullptr;
    if (!rc && (gate_bias || up_bias)) {
        std::vector<float> bi((size_t)rows, 0.0f);
        for (int64_t f = 0; f < F; ++f) {
            const int64_t r = (f / 128) * 256 + f % 128;
            if (gate_bias) bi[(size_t)r] = gate_bias[f];
            if (up_bias) bi[(size_t)(r + 128)] = up_bias[f];
        }
        rc = upload_bias(bi.data(), rows, &db);
    }
    if (!rc) {
        hipError_t e = hipStreamSynchronize(g.stream);
        if (e != hipSuccess) rc = fail(INV_ERR_HIP, "gate/up weight upload: %s", hipGetErrorString(e));
    }
    if (rc) {
        dev_free(dw);
        dev_free(db);
        return rc;
    }
    auto *h = new inv_weight_s{kWeightMagic, dw, db, F, K, ldw, 1, rows};
    g.weights.push_back(h);
    *out = h;
    return INV_OK;
}

int inv_hip_weight_free(inv_weight_t w) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!w) return INV_OK;
    if (!g.init) return fail(INV_ERR_NOT_INIT, "library not initialised");
    auto it = std::find(g.weights.begin(), g.weights.end(), w);
    if (it == g.weights.end()) return fail(INV_ERR_ARG, "unknown weight handle");
    (void)hipSetDevice(g.device);
    if (w->cached) {
        // a reference from inv_hip_weight_cache_get: the weight stays resident
        if (w->refs > 0) --w->refs;
        if (w->detached && w->refs == 0) {
            (void)hipStreamSynchronize(g.stream);
            drop_weight(w);
        } else {
            cache_trim();
        }
        return INV_OK;
    }
    (void)hipStreamSynchronize(g.stream);
    free_weight(w);
    g.weights.erase(it);
    return INV_OK;
}

int inv_hip_weight_cache_get(const char *path, const char *name, const char *bias_name, int flags,
                             inv_weight_t *out) {
    if (!out) return fail(INV_ERR_ARG, "weight cache: null output handle");
    *out = nullptr;
    if (!path || !name) return fail(INV_ERR_ARG, "weight cache: null path or tensor name");
    std::string key;
    TRY(cache_key(path, name, bias_name, flags, &key));
    {
        std::lock_guard<std::mutex> lk(g_mu);
        TRY(check_init());
        for (auto &e : g.cache)
            if (e.key == key) {
                ++e.w->refs;
                e.last_use = ++g.cache_clock;
                ++g.cache_hits;
                *out = e.w;
                return INV_OK;
            }
    }
    // A miss: load outside the lock (the upload takes it), then insert.
    inv_weight_t h = nullptr;
    TRY(inv_hip_weight_load_safetensors(path, name, bias_name, flags, &h));
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto &e : g.cache)
        if (e.key == key) {  // another thread loaded the same tensor meanwhile
            (void)hipStreamSynchronize(g.stream);
            drop_weight(h);
            ++e.w->refs;
            e.last_use = ++g.cache_clock;
            ++g.cache_hits;
            *out = e.w;
            return INV_OK;
        }
    h->cached = true;
    h->refs = 1;
    const size_t bytes = weight_bytes(h);
    g.cache.push_back({key, h, ++g.cache_clock, bytes});
    g.cache_bytes += bytes;
    ++g.cache_misses;
    g.cache_uploaded += (int64_t)bytes;
    cache_trim();
    *out = h;
    return INV_OK;
}

int inv_hip_weight_cache_set_budget(int64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (bytes < 0) return fail(INV_ERR_ARG, "weight cache: negative budget");
    g.cache_budget = bytes;
    cache_trim();
    return INV_OK;
}

int inv_hip_weight_cache_clear(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    (void)hipStreamSynchronize(g.stream);
    for (auto &e : g.cache) {
        if (e.w->refs == 0)
            drop_weight(e.w);
        else
            e.w->detached = true;  // freed by its last inv_hip_weight_free
    }
    g.cache.clear();
    g.cache_bytes = 0;
    return INV_OK;
}

int inv_hip_weight_cache_stats(int64_t *entries, int64_t *bytes, int64_t *hits, int64_t *misses,
                               int64_t *uploaded_bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (entries) *entries = (int64_t)g.cache.size();
    if (bytes) *bytes = (int64_t)g.cache_bytes;
    if (hits) *hits = g.cache_hits;
    if (misses) *misses = g.cache_misses;
    if (uploaded_bytes) *uploaded_bytes = g.cache_uploaded;
    return INV_OK;
}

int inv_hip_weight_shape(inv_weight_t w, int64_t *N, int64_t *K) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!valid_weight(w)) return fail(INV_ERR_ARG, "unknown weight handle");
    if (N) *N = w->N;
    if (K) *K = w->K;
    return INV_OK;
}

int inv_hip_linear(const void *X, int x_dtype, inv_weight_t W, const float *bias, void *Y, int y_dtype, int64_t M,
                   int64_t K, int64_t N, int epilogue, int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    return linear_impl("linear", X, x_dtype, W, bias, Y, y_dtype, M, K, N, epilogue, flags, false, nullptr);
}

int inv_hip_linear_noalloc(const void *X, int x_dtype, inv_weight_t W, const float *bias, void *Y, int y_dtype,
                           int64_t M, int64_t K, int64_t N, int epilogue, int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    return linear_noalloc_impl(X, x_dtype, W, bias, Y, y_dtype, M, K, N, epilogue, flags);
}

int inv_hip_linear_gated_add(const void *X, int x_dtype, inv_weight_t W, const float *bias, const float *gate,
                             float *Y, int64_t M, int64_t K, int64_t N, int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    return linear_impl("linear_gated_add", X, x_dtype, W, bias, Y, INV_DT_F32, M, K, N, INV_EPI_NONE, flags, true,
                       gate);
}

int inv_hip_linear_norm(const float *X, int norm, const float *norm_scale, const float *norm_shift, float eps,
                        inv_weight_t W, const float *bias, void *Y, int y_dtype, int64_t M, int64_t K, int64_t N,
                        int epilogue, int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (norm != INV_NORM_ADALN && norm != INV_NORM_RMS) return fail(INV_ERR_ARG, "linear_norm: bad norm %d", norm);
    if (norm == INV_NORM_ADALN && (!norm_scale || !norm_shift))
        return fail(INV_ERR_ARG, "linear_norm: AdaLN needs scale and shift");
    if (norm == INV_NORM_RMS && norm_shift) return fail(INV_ERR_ARG, "linear_norm: RMSNorm takes no shift");
    if (!(eps >= 0.0f) || eps > 3.0e38f) return fail(INV_ERR_ARG, "linear_norm: eps must be finite and >= 0");
    const NormArgs nm{norm, norm_scale, norm_shift, eps};
    return linear_impl("linear_norm", X, INV_DT_F32, W, bias, Y, y_dtype, M, K, N, epilogue, flags, false, nullptr, &nm);
}

int inv_hip_attention(const void *Q, const void *K, const void *V, void *O, int in_dtype, int out_dtype,
                      int64_t heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim, float scale,
                      int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    return attention_impl(Q, K, V, O, in_dtype, out_dtype, heads, kv_heads, seq_q, seq_k, head_dim, scale, nullptr,
                          flags);
}

int inv_hip_attention_masked(const void *Q, const void *K, const void *V, void *O, int in_dtype, int out_dtype,
                             int64_t heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                             float scale, const int32_t *key_mask, int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    return attention_impl(Q, K, V, O, in_dtype, out_dtype, heads, kv_heads, seq_q, seq_k, head_dim, scale, key_mask,
                          flags);
}

int inv_hip_head_norm_rope(float *X, int64_t seq, int64_t heads, int64_t head_dim, const float *norm_weight,
                           int rope, const float *cos_table, const float *sin_table, int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    return head_norm_rope_impl(X, seq, heads, head_dim, norm_weight, rope, cos_table, sin_table, flags);
}

int inv_hip_conv2d(const float *src, inv_weight_t weight, const float *bias, float *dst, int64_t in_ch, int64_t out_ch,
                   int64_t H, int64_t W, int64_t kH, int64_t kW, int64_t stride, int64_t padding, int64_t batch,
                   int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    return conv2d_impl(src, weight, bias, dst, in_ch, out_ch, H, W, kH, kW, stride, padding, batch, flags);
}

int inv_hip_attention_qk_norm_rope(const float *Q, int64_t ldq, const float *K, int64_t ldk, const float *V,
                                   int64_t ldv, void *O, int out_dtype, int64_t heads, int64_t kv_heads, int64_t seq_q,
                                   int64_t seq_k, int64_t head_dim, float scale, const float *q_norm_weight,
                                   const float *k_norm_weight, int rope, const float *q_cos, const float *q_sin,
                                   const float *k_cos, const float *k_sin, const int32_t *key_mask, int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    const int64_t hq = heads * head_dim, hk = kv_heads * head_dim;
    ldq = ldq ? ldq : hq;
    ldk = ldk ? ldk : hk;
    ldv = ldv ? ldv : hk;
    if (ldq < hq || ldk < hk || ldv < hk) return fail(INV_ERR_ARG, "attention: a leading dimension is below heads*head_dim");
    const QkPrep prep{q_norm_weight, k_norm_weight, rope, q_cos, q_sin, k_cos, k_sin, ldq, ldk, ldv};
    return attention_impl(Q, K, V, O, INV_DT_F32, out_dtype, heads, kv_heads, seq_q, seq_k, head_dim, scale, key_mask,
                          flags, &prep);
}

int inv_hip_set_sgemm_precision(int mode) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (mode != INV_PREC_BF16 && mode != INV_PREC_SPLIT_A && mode != INV_PREC_SPLIT_AB)
        return fail(INV_ERR_ARG, "bad precision mode %d", mode);
    g.sgemm_prec = mode;
    return INV_OK;
}

int inv_hip_sgemm(int order, int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                  int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc) {
    std::lock_guard<std::mutex> lk(g_mu);
    return gemm_slot(order, transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, INV_DT_F32);
}

int inv_hip_sbgemm(int order, int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const uint16_t *A,
                   int64_t lda, const uint16_t *B, int64_t ldb, float beta, float *C, int64_t ldc) {
    std::lock_guard<std::mutex> lk(g_mu);
    return gemm_slot(order, transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, INV_DT_BF16);
}

int inv_hip_malloc(void **ptr, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!ptr) return fail(INV_ERR_ARG, "malloc: null out pointer");
    return dev_alloc(ptr, std::max<size_t>(bytes, 1), "malloc");
}

int inv_hip_free(void *ptr) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!ptr) return INV_OK;
    HIPCHK(hipStreamSynchronize(g.stream));
    if (!g.allocs.count(ptr)) return fail(INV_ERR_ARG, "free: %p was not allocated by inv_hip_malloc", ptr);
    dev_free(ptr);
    return INV_OK;
}

int inv_hip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!bytes) return INV_OK;
    if (!dst || !src) return fail(INV_ERR_ARG, "memcpy_h2d: null pointer");
    TRY(h2d_rows(dst, src, 1, bytes, bytes));
    HIPCHK(hipStreamSynchronize(g.stream));
    return INV_OK;
}

int inv_hip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!bytes) return INV_OK;
    if (!dst || !src) return fail(INV_ERR_ARG, "memcpy_d2h: null pointer");
    return d2h_rows(dst, src, 1, bytes, bytes);
}

int inv_hip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!bytes) return INV_OK;
    if (!dst || !src) return fail(INV_ERR_ARG, "memcpy_d2d: null pointer");
    if (aligned(dst, 16) && aligned(src, 16) && bytes % 16 == 0) {
        const int64_t n16 = (int64_t)(bytes / 16);
        const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, (int64_t)g.cu_count * 16);
        hipLaunchKernelGGL(inv::copy_words16, dim3((unsigned)blocks), dim3(256), 0, g.stream, (const uint4 *)src,
                           (uint4 *)dst, n16);
        HIPCHK(hipGetLastError());
    } else {
        HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g.stream));
    }
    HIPCHK(hipStreamSynchronize(g.stream));
    return INV_OK;
}

int inv_hip_memset(void *dst, int value, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!bytes) return INV_OK;
    if (!dst) return fail(INV_ERR_ARG, "memset: null pointer");
    HIPCHK(hipMemsetAsync(dst, value, bytes, g.stream));
    HIPCHK(hipStreamSynchronize(g.stream));
    return INV_OK;
}

int inv_hip_synchronize(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    HIPCHK(hipStreamSynchronize(g.stream));
    return INV_OK;
}

int inv_hip_timer_start(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    HIPCHK(hipEventRecord(g.tim0, g.stream));
    return INV_OK;
}

int inv_hip_timer_stop(float *ms) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    if (!ms) return fail(INV_ERR_ARG, "timer_stop: null pointer");
    HIPCHK(hipEventRecord(g.tim1, g.stream));
    HIPCHK(hipEventSynchronize(g.tim1));
    HIPCHK(hipEventElapsedTime(ms, g.tim0, g.tim1));
    return INV_OK;
}

int inv_hip_stats_enable(int enable) {
    std::lock_guard<std::mutex> lk(g_mu);
    TRY(check_init());
    g.stats = enable != 0;
    return INV_OK;
}

int inv_hip_stats(int64_t *calls, double *gemm_ms, double *flops) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (calls) *calls = g.calls;
    if (gemm_ms) *gemm_ms = g.gemm_ms;
    if (flops) *flops = g.flops;
    return INV_OK;
}

int inv_hip_stats_reset(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    g.calls = 0;
    g.gemm_ms = g.flops = 0.0;
    return INV_OK;
}

}  // extern "C"
