// engine.hip -- the C-ABI launch layer (include/msplat_engine.h): one HIP
// stream, a cache of intermediate device buffers that grows on demand, and
// the stage sequencing of the reference's msplat_train_step_2dgs /
// msplat_render / msplat_fused_adam / msplat_densify
// (core/metal/msplat_metal.mm:545-1594).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <exception>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.h"
#include "msplat_engine.h"

// host side (host/hostcopy.cpp): memcpy split over a few OpenMP threads
void ms_parallel_memcpy(void *dst, const void *src, size_t bytes);

// Scratch of msplat_hip_loss_fwd_bwd_noalloc, for callers that cannot
// allocate: the three per-pixel SSIM partial maps (12 B per pixel each, at
// fixed offsets sized for kNoAllocMaxPixels), then the per-workgroup loss
// partials (16 B per 32x32 tile, kNoAllocMaxBlocks of them), then the two
// loss doubles.  Every call on a GPU shares that GPU's copy and leaves its
// contents behind; each call rewrites every element it later reads, so
// nothing needs clearing.  In host code `scratch` is only a symbol: kernels
// get the device address from hipGetSymbolAddress (g_scratch_dev).
constexpr int64_t kNoAllocMaxPixels = int64_t(1) << 21;  // e.g. 2048 x 1024, 1920 x 1080
constexpr int64_t kNoAllocMaxBlocks = int64_t(1) << 17;
constexpr size_t kNoAllocMapBytes = (size_t)kNoAllocMaxPixels * 12;
constexpr size_t kNoAllocPartialsOff = 3 * kNoAllocMapBytes;
constexpr size_t kNoAllocLossOff = kNoAllocPartialsOff + (size_t)kNoAllocMaxBlocks * 16;
constexpr size_t kNoAllocBytes = kNoAllocLossOff + 256;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

constexpr int kMaxDevices = 64;
void *g_scratch_dev[kMaxDevices] = {};  // device address of `scratch`, per device

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

enum StageId { ST_PROJECT, ST_SCAN, ST_SCATTER_SORT, ST_RASTER_FWD, ST_LOSS, ST_RASTER_BWD, ST_PROJECT_BWD, ST_COUNT };
const char *kStageNames[ST_COUNT] = {"project_fwd", "tile_scan", "scatter_sort", "raster_fwd",
                                     "ssim_l1",     "raster_bwd", "project_bwd_adam"};

constexpr size_t kD2HChunk = size_t(8) << 20;  // bytes per pinned download chunk

// Deep-tile threshold: no tile of the 500k and 3M-splat blob workloads holds
// more than 3.3k entries; the overflow workload's cluster tiles hold up to 200k.
// By default a deep tile also holds 4x the frame's mean list: the deep path's
// per-pixel lists and log rebuild pay off only for lists far above the rest
// (measured: the densify workload's end, 62 tiles of 4.4k-5.3k entries against
// a 1.6k mean, trains 4% faster with them per tile; the overflow workload's
// forward slows from 0.65 to 0.68 ms with a 6144 threshold instead of 4096).
constexpr int kDefaultDeepLen = 4096;
constexpr int kDeepMeanFactor = 4;

struct Engine {
    bool ready = false;
    int device = 0;
    hipStream_t stream = nullptr;
    int *pinned_i = nullptr;     // small pinned readback area
    int *pinned_ctr = nullptr;   // the blend-log pool's counters
    double *pinned_d = nullptr;
    // two pinned chunks of kD2HChunk bytes for large downloads (RGBA8
    // frames) and the events of their DMAs
    unsigned char *stage = nullptr;
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
    float window[11];
    // per-gaussian
    // rec: N splat records (MSPLAT_REC_FLOATS each), followed by their N
    // quadrant-mask records (msd::MaskRec, 12 floats each; mask_recs())
    DevBuf rec, depths, radii, rect, grads16, colors_raw;
    // per-tile
    DevBuf counts, offsets, stats, big_list, scan_tmp;
    DevBuf huge_list, chunk_base, chunk_counts;  // the longest super-tile lists, their chunk numbering and counts
    DevBuf merge_base;                           // the merge-tile numbering of the lists above 4096 keys
    DevBuf super_counts, super_offsets, super_cm, super_tmp;  // super_cm: per-(workgroup, super-tile) offsets
    // per-intersection
    DevBuf keys, keys_tmp, ids;  // keys: per (splat, super-tile) pair
    DevBuf blend_log, t_ckpt, wave_cnt;  // the raster forward's per-wave blend log
    DevBuf selfcheck;                    // counter of the arithmetic self-check
    // per-pixel
    DevBuf out_img, final_Ts, final_idx, out_depth, out_normal, out_alpha, out_median, out_dist;
    DevBuf dL_dimg, gm1, gs1, gs12, partials, loss;
    // unfused gradients
    DevBuf dmeans, dscales, dquats, dmean2d, dfdc, dfrest;
    // materialised views
    DevBuf mat[MSPLAT_LAST_COUNT];
    // densify scratch
    DevBuf dens_ws, dens_flags, dens_scan, dens_keep;
    int64_t dens_rows = 0;  // rows dens_ws and dens_keep are sized for
    DevBuf pair_counter;
    DevBuf rgba;  // RGBA8 staging of msplat_hip_image_to_rgba8
    // mesh extraction: TSDF view records and pixel masks, marching-cubes case
    // bytes, and the per-chunk counts / scanned offsets of the two compactions
    DevBuf tsdf_views, tsdf_masks, mc_cases, chunk_cnt, chunk_off;
    // state of the most recent forward
    int n = 0, W = 0, H = 0, tiles_x = 0, tiles_y = 0, K3 = 0;
    int64_t num_isect = 0;
    const float *bg = nullptr;
    bool have_grads = false;
    bool raster_grads = false;  // grads16 belongs to the current forward
    bool g16_moments = false;   // grads16 holds the image-only backward's unfinished sums
    bool gs3d = false;        // the most recent forward is the 3DGS mode's
    bool log_valid = false;   // blend log written for the most recent forward
    bool full_valid = false;  // depth / normal / alpha / median / distortion outputs written
    // timing
    bool timing = false;       // HIP events per stage
    bool count_pairs = false;  // raster pair counter
    bool defer_deep_log = false;  // set by the training step around its forward
    bool wide_keys = false;    // binning test hook: the wide key layout at any N
    // tiles whose list holds at least deep_frame entries are rendered pixel
    // by pixel (mskern::DeepTiles); n_deep of them in the current frame.
    // deep_frame is deep_len when a test set it (deep_len_set), else the
    // larger of deep_len and kDeepMeanFactor x the frame's mean list
    int deep_len = kDefaultDeepLen, deep_frame = kDefaultDeepLen, n_deep = 0;
    bool deep_len_set = false;
    DevBuf deep_list, deep_pos, deep_tb, deep_cnt;
    // blend-log pool (msr::BlendLog): blend_log / t_ckpt hold log_used chunks
    // of 64 entries / checkpoints, log_table the per-wave chunk tables,
    // log_ctr the sub-pool and spill counters and the overflow flag
    DevBuf log_table, log_ctr;
    int64_t log_cap = 0;   // the size overflows grew the pool to
    int64_t log_used = 0;  // chunks of the current frame's pool
    int64_t log_init = 0;  // estimate override in chunks (0: from the frame)
    int64_t log_redos = 0; // overflowed logs since init
    int64_t log_demand = 0;  // chunks the last fitting log claimed
    // the largest demand / static estimate seen, per mode (2DGS, 3DGS):
    // their splats cover tiles differently
    double log_fill[2] = {0.0, 0.0};
    msr::BlendLog log_desc{};  // the current frame's pool layout
    hipStream_t deep_stream = nullptr;  // default priority, non-blocking
    hipEvent_t deep_fork = nullptr, deep_join = nullptr, deep_logged = nullptr;
    hipEvent_t ev[ST_COUNT + 1] = {};
    float stage_ms[ST_COUNT] = {};
    bool stage_valid[ST_COUNT] = {};
    int64_t pairs[5] = {0, 0, 0, 0, 0};  // evaluated, log entries, blended, visits, visit slots
};

Engine g_eng;
std::mutex g_mu;
char g_err[1024] = "";

void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

#define HIPC(expr)                                                                        \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess) {                                                           \
            set_err("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
            return MSPLAT_E_HIP;                                                          \
        }                                                                                 \
    } while (0)

#define CHECK(expr)                   \
    do {                              \
        int r_ = (expr);              \
        if (r_ != MSPLAT_OK) return r_; \
    } while (0)

int ensure(DevBuf &b, size_t bytes) {
    if (bytes == 0) bytes = 16;
    if (b.cap >= bytes) return MSPLAT_OK;
    if (b.p) HIPC(hipFree(b.p));
    b.p = nullptr;
    b.cap = 0;
    const size_t want = bytes + bytes / 8;  // headroom against small growth
    if (hipMalloc(&b.p, want) != hipSuccess) {
        (void)hipGetLastError();
        set_err("hipMalloc(%zu bytes) failed", want);
        b.p = nullptr;
        return MSPLAT_E_NOMEM;
    }
    b.cap = want;
    return MSPLAT_OK;
}

template <typename T>
T *P(DevBuf &b) {
    return static_cast<T *>(b.p);
}

// The quadrant-mask records of the current frame's E.n splats, stored after
// their splat records in E.rec.
float *mask_recs() { return P<float>(g_eng.rec) + (size_t)g_eng.n * MSPLAT_REC_FLOATS; }

int check_rcp_locked(int lo, int hi, int64_t *bad);

int init_locked() {
    if (g_eng.ready) return MSPLAT_OK;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        set_err("no HIP device available");
        return MSPLAT_E_NODEV;
    }
    if (g_eng.device < 0 || g_eng.device >= kMaxDevices) {
        set_err("device %d out of range", g_eng.device);
        return MSPLAT_E_NODEV;
    }
    HIPC(hipSetDevice(g_eng.device));
    hipDeviceProp_t prop;
    HIPC(hipGetDeviceProperties(&prop, g_eng.device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err("device arch %s is not gfx950", prop.gcnArchName);
        return MSPLAT_E_NODEV;
    }
    HIPC(hipStreamCreateWithFlags(&g_eng.stream, hipStreamNonBlocking));
    HIPC(hipHostMalloc((void **)&g_eng.pinned_i, 64 * sizeof(int), hipHostMallocDefault));
    HIPC(hipHostMalloc((void **)&g_eng.pinned_ctr, 264 * sizeof(int), hipHostMallocDefault));
    HIPC(hipHostMalloc((void **)&g_eng.pinned_d, 16 * sizeof(double), hipHostMallocDefault));
    HIPC(hipHostMalloc((void **)&g_eng.stage, 2 * kD2HChunk, hipHostMallocDefault));
    for (auto &e : g_eng.stage_ev) HIPC(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    for (int i = 0; i <= ST_COUNT; ++i) HIPC(hipEventCreate(&g_eng.ev[i]));
    // this device's copy of the no-allocation entry point's scratch array
    if (!g_scratch_dev[g_eng.device]) {
        void *sp = nullptr;
        HIPC(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
        if (!sp) {
            set_err("hipGetSymbolAddress(scratch) returned no address");
            return MSPLAT_E_HIP;
        }
        g_scratch_dev[g_eng.device] = sp;
    }
    // The 11-tap SSIM window exp(-(x-5)^2 / 4.5) / sum (the table of
    // msplat_metal.metal:2804-2816), evaluated in double and rounded once.
    double gsum = 0.0, gw[11];
    for (int i = 0; i < 11; ++i) {
        const double d = i - 5.0;
        gw[i] = std::exp(-d * d / (2.0 * 1.5 * 1.5));
        gsum += gw[i];
    }
    for (int i = 0; i < 11; ++i) g_eng.window[i] = (float)(gw[i] / gsum);
    // The rasterizer takes 1 / ray.z as the hardware reciprocal plus one
    // Newton step, which must equal the correctly rounded division (the
    // golden model's); verified here over [1, 2) and (-2, -1].
    int64_t bad = 0;
    CHECK(check_rcp_locked(127, 127, &bad));
    if (bad != 0) {
        set_err("fast reciprocal differs from division on %lld floats of [1, 2)", (long long)bad);
        return MSPLAT_E_NODEV;
    }
    g_eng.ready = true;
    return MSPLAT_OK;
}

// Floats of exponent fields lo..hi where the rasterizer's fast reciprocal
// differs from the correctly rounded division (synchronous).
int check_rcp_locked(int lo, int hi, int64_t *bad) {
    Engine &E = g_eng;
    CHECK(ensure(E.selfcheck, 8));
    HIPC(hipMemsetAsync(E.selfcheck.p, 0, 8, E.stream));
    for (int ef = lo; ef <= hi; ++ef) mskern::launch_check_rcp(E.stream, ef, P<unsigned long long>(E.selfcheck));
    HIPC(hipGetLastError());
    unsigned long long h = 0;
    HIPC(hipMemcpyAsync(&h, E.selfcheck.p, 8, hipMemcpyDeviceToHost, E.stream));
    HIPC(hipStreamSynchronize(E.stream));
    *bad = (int64_t)h;
    return MSPLAT_OK;
}

#define ENSURE_INIT()                      \
    do {                                   \
        int r0_ = init_locked();           \
        if (r0_ != MSPLAT_OK) return r0_;  \
    } while (0)

void stage_mark(int s) {
    if (g_eng.timing) (void)hipEventRecord(g_eng.ev[s], g_eng.stream);
}

int validate_cam(const MsplatCamera *cam, const MsplatGaussians *g) {
    if (!cam || !g) {
        set_err("null camera or gaussians");
        return MSPLAT_E_ARG;
    }
    if (cam->width <= 0 || cam->height <= 0 || cam->tiles_x != (cam->width + 15) / 16 ||
        cam->tiles_y != (cam->height + 15) / 16 || cam->tiles_x > 65535 || cam->tiles_y > 65535) {
        set_err("invalid image size %dx%d / tiles %dx%d", cam->width, cam->height, cam->tiles_x, cam->tiles_y);
        return MSPLAT_E_ARG;
    }
    if (cam->degree < 0 || cam->degree > 4 || cam->degrees_to_use < 0 || cam->degrees_to_use > cam->degree) {
        set_err("invalid SH degree %d / degrees_to_use %d", cam->degree, cam->degrees_to_use);
        return MSPLAT_E_ARG;
    }
    if (g->num_points < 0 ||
        (g->num_points > 0 && (!g->means || !g->scales || !g->quats || !g->opacities || !g->features_dc ||
                               (cam->degree > 0 && !g->features_rest)))) {
        set_err("invalid gaussian buffers");
        return MSPLAT_E_ARG;
    }
    return MSPLAT_OK;
}

// Stages a3-a7: projection, binning, per-tile sort, rasterize forward.
// With log, the raster forward also writes the blend log the backward
// replays; with full, it also produces the depth, normal, alpha, median and
// distortion outputs.  The forward is deterministic, so running it again on
// the same tile lists (to add the log or the full outputs on demand)
// reproduces every value it wrote before.
// The current frame's deep tiles (none in the 3DGS mode), with the stream
// and events their kernels run between.
int deep_tiles(mskern::DeepTiles &deep) {
    Engine &E = g_eng;
    deep = mskern::DeepTiles{};
    if (E.n_deep <= 0 || E.gs3d) return MSPLAT_OK;
    if (!E.deep_stream) {
        HIPC(hipStreamCreateWithFlags(&E.deep_stream, hipStreamNonBlocking));
        HIPC(hipEventCreateWithFlags(&E.deep_fork, hipEventDisableTiming));
        HIPC(hipEventCreateWithFlags(&E.deep_join, hipEventDisableTiming));
        HIPC(hipEventCreateWithFlags(&E.deep_logged, hipEventDisableTiming));
    }
    deep.n = E.n_deep;
    deep.len = E.deep_frame;
    deep.list = P<int>(E.deep_list);
    deep.stream = E.deep_stream;
    deep.fork = E.deep_fork;
    deep.join = E.deep_join;
    deep.logged = E.deep_logged;
    return MSPLAT_OK;
}

// The most chunks the frame's logs can take: every wave's ceil(len / 64).
int64_t log_worst_chunks(const Engine &E) { return 4 * (int64_t)E.num_isect / 64 + 4 * (int64_t)E.tiles_x * E.tiles_y; }
int log_subpools(int64_t tiles) { return (int)std::min<int64_t>(256, std::max<int64_t>(1, tiles / 64)); }
// One chunk per 96 intersections plus a partial chunk per wave.
int64_t log_static_estimate(const Engine &E) {
    return std::max<int64_t>(1024, (int64_t)E.num_isect / 96 + 4 * (int64_t)E.tiles_x * E.tiles_y);
}
// The largest pool: a spill region of the worst case (no log can overflow
// it, whatever the sub-pools' shares) beside sub-pools of three quarters
// of it.
int64_t log_max_chunks(const Engine &E) {
    const int64_t worst = log_worst_chunks(E);
    return worst + 3 * worst / 4 + log_subpools((int64_t)E.tiles_x * E.tiles_y);
}

// The frame's blend-log pool of `cap` chunks: a sub-pool per 64 tiles (at
// most 256; wave w of tile t claims from sub-pool (4t + w) mod count) takes
// three quarters, the spill region the rest, and the largest pool a spill
// region of the worst case.  cap is the larger of the frame's estimate and
// the size earlier overflows grew the pool to (log_cap), at most the
// largest pool.  The estimate is a static one (about a sixth of the worst
// case; the training step at 3M splats claims 45-62% of it) until a log
// fitted, then that scaled by 1.25 times the largest ratio of claimed chunks
// to it seen so far in the frame's mode (log_fill).  A step whose log overflows is redone
// after the pool grows (grow_log_pool).  Planned by each forward that logs;
// the backward reads the log through the plan kept in log_desc.
int plan_log_pool(msr::BlendLog &L) {
    Engine &E = g_eng;
    const int64_t T = (int64_t)E.tiles_x * E.tiles_y;
    const int64_t worst = log_worst_chunks(E), most = log_max_chunks(E);
    if (most > INT32_MAX / 2) {
        set_err("blend log: too many intersections for the pool's chunk indices");
        return MSPLAT_E_ARG;
    }
    const int64_t base = log_static_estimate(E);
    const double fill = E.log_fill[E.gs3d];
    const int64_t estimate = E.log_init          ? E.log_init
                             : fill > 0.0       ? std::max<int64_t>(1024, (int64_t)std::ceil(1.25 * fill * (double)base))
                                                : base;
    const int64_t cap = std::min(std::max(E.log_cap, estimate), most);
    E.log_used = cap;
    CHECK(ensure(E.blend_log, (size_t)cap * 64 * mskern::kBlendLogEntryBytes));
    CHECK(ensure(E.t_ckpt, (size_t)cap * 64 * 4));
    CHECK(ensure(E.log_table, msr::log_table_ints(E.num_isect, (int)T) * 4));
    CHECK(ensure(E.wave_cnt, (size_t)4 * T * 4));
    const int nsub = log_subpools(T);
    const int64_t spill = cap == most ? worst : cap / 4;
    CHECK(ensure(E.log_ctr, (size_t)(nsub + 2) * 4));
    L.ent = P<uint4>(E.blend_log);
    L.ckpt = P<float>(E.t_ckpt);
    L.table = P<int>(E.log_table);
    L.wave_cnt = P<int>(E.wave_cnt);
    L.counters = P<int>(E.log_ctr);
    L.overflow = P<int>(E.log_ctr) + nsub + 1;
    L.nsub = nsub;
    L.sub_cap = (int)((cap - spill) / nsub);
    L.spill_cap = (int)spill;
    E.log_desc = L;
    return MSPLAT_OK;
}

// Queues the copy of the pool's counters and overflow flag after a logging
// forward; once the stream has synchronised, log_account returns whether
// the log overflowed and, if not, records the frame's demand (each claim is
// counted in its sub-pool's counter, also when the spill region served it).
int log_readback(const msr::BlendLog &L, hipStream_t s) {
    HIPC(hipMemcpyAsync(g_eng.pinned_ctr, L.counters, (size_t)(L.nsub + 2) * 4, hipMemcpyDeviceToHost, s));
    return MSPLAT_OK;
}
bool log_account(const msr::BlendLog &L) {
    Engine &E = g_eng;
    if (g_eng.pinned_ctr[L.nsub + 1] != 0) return true;
    int64_t demand = 0;
    for (int i = 0; i < L.nsub; ++i) demand += g_eng.pinned_ctr[i];
    E.log_demand = demand;
    double &fill = E.log_fill[E.gs3d];
    fill = std::max(fill, (double)demand / (double)log_static_estimate(E));
    return false;
}

// Zeroes the pool's counters and overflow flag before a forward that logs.
int reset_log_pool(const msr::BlendLog &L) {
    HIPC(hipMemsetAsync(L.counters, 0, (size_t)(L.nsub + 2) * 4, g_eng.stream));
    return MSPLAT_OK;
}

// After an overflowed log: a pool 1.5 times as large as the one that
// overflowed, at most the largest (in which no log overflows).
void grow_log_pool() {
    Engine &E = g_eng;
    E.log_cap = std::min(log_max_chunks(E), std::max<int64_t>(E.log_used + E.log_used / 2, 64));
    E.log_valid = false;
    ++E.log_redos;
}

int raster_fwd_locked(bool log, bool full) {
    Engine &E = g_eng;
    msr::BlendLog blog{};
    mskern::DeepTiles deep;
    CHECK(deep_tiles(deep));
    if (deep.n > 0) {
        if (log) {
            const size_t ent = (size_t)mskern::deep_pixel_entries(E.n_deep);
            CHECK(ensure(E.deep_pos, ent * 4));
            CHECK(ensure(E.deep_tb, ent * 4));
            CHECK(ensure(E.deep_cnt, (size_t)E.n_deep * 256 * 4));
            deep.pos = P<int>(E.deep_pos);
            deep.tb = P<float>(E.deep_tb);
            deep.cnt = P<int>(E.deep_cnt);
        }
    }
    if (log) {
        CHECK(plan_log_pool(blog));
        CHECK(reset_log_pool(blog));
    }
    deep.defer_log = log && E.defer_deep_log;
    if (E.gs3d) {
        if (full) {
            set_err("the 3DGS mode produces the image and the transmittance only");
            return MSPLAT_E_ARG;
        }
        mskern::launch_raster3d_fwd(E.stream, E.W, E.H, E.tiles_x, E.tiles_y, P<int>(E.offsets), P<int>(E.ids),
                                    P<float>(E.rec), P<float>(E.rec) + (size_t)E.n * mskern::kRec3Floats, E.bg,
                                    P<float>(E.out_img), P<float>(E.final_Ts), log ? &blog : nullptr);
        E.log_valid = E.log_valid || log;
        return MSPLAT_OK;
    }
    mskern::launch_raster_fwd(E.stream, E.W, E.H, E.tiles_x, E.tiles_y, P<int>(E.offsets), P<int>(E.ids),
                              P<float>(E.rec), mask_recs(), E.bg, P<float>(E.out_img), P<float>(E.final_Ts),
                              P<int>(E.final_idx),
                              P<float>(E.out_depth), P<float>(E.out_normal), P<float>(E.out_alpha),
                              P<float>(E.out_median), P<float>(E.out_dist),
                              E.count_pairs ? P<unsigned long long>(E.pair_counter) : nullptr, log ? &blog : nullptr,
                              full, deep);
    E.log_valid = E.log_valid || log;
    E.full_valid = E.full_valid || full;
    return MSPLAT_OK;
}

// A forward replay with the blend log outside the training step: waits for
// it and replays again with a larger pool until the log fits.
int log_forward_checked(bool full) {
    Engine &E = g_eng;
    for (;;) {
        CHECK(raster_fwd_locked(true, full));
        CHECK(log_readback(E.log_desc, E.stream));
        HIPC(hipStreamSynchronize(E.stream));
        if (!log_account(E.log_desc)) return MSPLAT_OK;
        grow_log_pool();
    }
}

int forward_locked(const MsplatCamera *cam, const MsplatGaussians *g, const float *bg, int64_t *nisect, bool log,
                   bool full, bool gs3d = false) {
    CHECK(validate_cam(cam, g));
    if (!bg) {
        set_err("null background");
        return MSPLAT_E_ARG;
    }
    Engine &E = g_eng;
    hipStream_t s = E.stream;
    const int N = g->num_points, W = cam->width, H = cam->height;
    const int T = cam->tiles_x * cam->tiles_y;
    const size_t Pn = (size_t)W * H;
    const int nb = cam->degree == 0 ? 1 : cam->degree == 1 ? 4 : cam->degree == 2 ? 9 : cam->degree == 3 ? 16 : 25;
    CHECK(ensure(E.rec, (size_t)N * (MSPLAT_REC_FLOATS + 12) * 4));
    CHECK(ensure(E.depths, (size_t)N * 4));
    CHECK(ensure(E.radii, (size_t)N * 4));
    CHECK(ensure(E.rect, (size_t)N * 8));
    CHECK(ensure(E.counts, (size_t)T * 4));
    CHECK(ensure(E.scan_tmp, (size_t)mskern::tile_scan_temp_ints(T) * 4));
    CHECK(ensure(E.offsets, (size_t)(T + 1) * 4));
    const int sxn = (cam->tiles_x + mskern::kSuperTile - 1) / mskern::kSuperTile;
    const int syn = (cam->tiles_y + mskern::kSuperTile - 1) / mskern::kSuperTile;
    const int NS = sxn * syn;
    CHECK(ensure(E.super_counts, (size_t)NS * 4));
    CHECK(ensure(E.super_offsets, (size_t)(NS + 1) * 4));
    CHECK(ensure(E.super_cm, (size_t)mskern::kBinMaxBlocks * NS * 4));
    CHECK(ensure(E.super_tmp, (size_t)mskern::tile_scan_temp_ints(NS) * 4));
    // stats (ints): [0..1] tiles: total, largest; [4..7] super-tiles: total,
    // largest, long lists, their merge tiles; [8..9] 64-bit intersection
    // count from the projection; [12..13] huge lists, their chunks; [14]
    // deep tiles
    CHECK(ensure(E.stats, 64));
    CHECK(ensure(E.big_list, (size_t)NS * 4));
    CHECK(ensure(E.out_img, Pn * 12));
    CHECK(ensure(E.final_Ts, Pn * 12));
    CHECK(ensure(E.final_idx, Pn * 8));
    CHECK(ensure(E.out_depth, Pn * 4));
    CHECK(ensure(E.out_normal, Pn * 12));
    CHECK(ensure(E.out_alpha, Pn * 4));
    CHECK(ensure(E.out_median, Pn * 4));
    CHECK(ensure(E.out_dist, Pn * 4));
    CHECK(ensure(E.pair_counter, 40));
    E.n = N;
    E.W = W;
    E.H = H;
    E.tiles_x = cam->tiles_x;
    E.tiles_y = cam->tiles_y;
    E.K3 = (nb - 1) * 3;
    E.bg = bg;
    E.have_grads = false;
    E.raster_grads = false;
    E.g16_moments = false;
    E.log_valid = false;
    E.full_valid = false;
    E.gs3d = gs3d;
    for (int i = 0; i < ST_COUNT; ++i) E.stage_valid[i] = false;

    stage_mark(ST_PROJECT);
    HIPC(hipMemsetAsync(E.stats.p, 0, 64, s));
    if (E.count_pairs) HIPC(hipMemsetAsync(E.pair_counter.p, 0, 40, s));
    // the 3DGS rasterizers count nothing: no counters for this forward
    if (gs3d) std::fill(E.pairs, E.pairs + 5, int64_t(0));
    if (gs3d)
        mskern::launch_project3d_fwd(s, *cam, *g, P<float>(E.rec), P<float>(E.rec) + (size_t)N * mskern::kRec3Floats,
                                     P<float>(E.depths), P<int>(E.radii), P<uint32_t>(E.rect),
                                     reinterpret_cast<unsigned long long *>(P<int>(E.stats) + 8), nullptr);
    else
        mskern::launch_project_fwd(s, *cam, *g, P<float>(E.rec), mask_recs(), P<float>(E.depths), P<int>(E.radii),
                                   P<uint32_t>(E.rect), reinterpret_cast<unsigned long long *>(P<int>(E.stats) + 8),
                                   nullptr);
    stage_mark(ST_SCAN);
    mskern::launch_super_count(s, N, cam->tiles_x, cam->tiles_y, P<int>(E.radii), P<uint32_t>(E.rect),
                               P<int>(E.super_counts), P<int>(E.super_offsets), P<int>(E.super_cm),
                               P<int>(E.stats) + 4, P<int>(E.super_tmp));
    HIPC(hipMemcpyAsync(E.pinned_i, E.stats.p, 16 * sizeof(int), hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
    unsigned long long isect64;
    std::memcpy(&isect64, E.pinned_i + 8, sizeof(isect64));
    const int S_total = E.pinned_i[4], super_max = E.pinned_i[5];
    if (isect64 > 0x7fffffffull || S_total < 0) {
        set_err("tile intersection count %llu overflows int32", isect64);
        return MSPLAT_E_CAPACITY;
    }
    const int I = (int)isect64;
    E.num_isect = I;
    if (nisect) *nisect = I;
    stage_mark(ST_SCATTER_SORT);
    CHECK(ensure(E.keys, (size_t)S_total * 8));
    CHECK(ensure(E.ids, (size_t)I * 4));
    if (super_max > mskern::kSuperSortChunk) {
        CHECK(ensure(E.keys_tmp, (size_t)S_total * 8));
        CHECK(ensure(E.merge_base, (size_t)NS * 4));
    }
    if (mskern::bin_chunk_parallel(super_max, NS)) {
        CHECK(ensure(E.huge_list, (size_t)NS * 4));
        CHECK(ensure(E.chunk_base, (size_t)NS * 4));
        CHECK(ensure(E.chunk_counts, (size_t)mskern::big_chunk_ints(S_total, NS) * 4));
    }
    E.deep_frame = E.deep_len_set ? E.deep_len
                                  : (int)std::max<int64_t>(E.deep_len, kDeepMeanFactor * (int64_t)I / T);
    // a tile's list is at most its super-tile's: no deep tile below that
    const bool scan_deep = !gs3d && super_max >= E.deep_frame;
    mskern::DeepScan dscan;
    if (scan_deep) {
        CHECK(ensure(E.deep_list, (size_t)T * 4));
        dscan.len = E.deep_frame;
        dscan.list = P<int>(E.deep_list);
        dscan.count = P<int>(E.stats) + 14;
        dscan.host_count = E.pinned_i + 14;
    }
    mskern::launch_bin_tiles(s, N, cam->tiles_x, cam->tiles_y, P<int>(E.radii), P<uint32_t>(E.rect),
                             P<float>(E.depths), P<int>(E.super_offsets), P<int>(E.super_cm), super_max,
                             P<uint64_t>(E.keys), P<uint64_t>(E.keys_tmp), P<int>(E.big_list), P<int>(E.stats) + 4,
                             P<int>(E.huge_list), P<int>(E.stats) + 12, P<int>(E.chunk_base), P<int>(E.chunk_counts),
                             P<int>(E.merge_base), S_total, P<int>(E.counts), P<int>(E.offsets), P<int>(E.stats),
                             P<int>(E.scan_tmp), P<int>(E.ids), E.wide_keys, scan_deep ? &dscan : nullptr);
    E.n_deep = 0;
    if (scan_deep) {
        HIPC(hipStreamSynchronize(s));
        E.n_deep = E.pinned_i[14];
    }
    stage_mark(ST_RASTER_FWD);
    CHECK(raster_fwd_locked(log, full));
    HIPC(hipGetLastError());
    return MSPLAT_OK;
}

int loss_locked(int W, int H, const float *img, const float *gt, const float *dist, float l1, float ldist,
                float ldssim, float *dL) {
    Engine &E = g_eng;
    if (mskern::loss_needs_maps(W, H)) {
        const size_t E3 = (size_t)W * H * 3;
        CHECK(ensure(E.gm1, E3 * 4));
        CHECK(ensure(E.gs1, E3 * 4));
        CHECK(ensure(E.gs12, E3 * 4));
    }
    CHECK(ensure(E.partials, (size_t)mskern::loss_num_partials(W, H) * 16));
    CHECK(ensure(E.loss, 16));
    mskern::launch_loss_fwd_bwd(E.stream, W, H, img, gt, dist, l1, ldist, ldssim, E.window, P<float>(E.gm1),
                                P<float>(E.gs1), P<float>(E.gs12), P<double>(E.partials), P<double>(E.loss), dL);
    HIPC(hipGetLastError());
    return MSPLAT_OK;
}

int last_locked(int which, void **ptr, int64_t *numel) {
    Engine &E = g_eng;
    *ptr = nullptr;
    *numel = 0;
    switch (which) {
        case MSPLAT_LAST_FINAL_TS:
            if (E.gs3d) break;  // the transmittance (its first component) is written by every 3DGS forward
            [[fallthrough]];
        case MSPLAT_LAST_FINAL_IDX: case MSPLAT_LAST_OUT_DEPTH:
        case MSPLAT_LAST_OUT_NORMAL: case MSPLAT_LAST_OUT_ALPHA: case MSPLAT_LAST_OUT_MEDIAN_DEPTH:
        case MSPLAT_LAST_OUT_DISTORTION:
            // produced on demand after an image-only forward
            if (E.rec.p && !E.full_valid) CHECK(raster_fwd_locked(false, true));
            break;
        case MSPLAT_LAST_GRADS16: case MSPLAT_LAST_DL_DTRANSMAT: case MSPLAT_LAST_DL_DNORMAL3D:
        case MSPLAT_LAST_DL_DOPACITY: case MSPLAT_LAST_DL_DCOLORS:
            if (!E.raster_grads) return MSPLAT_OK;  // none for the current forward
            // the image-only backward leaves ray moments; turn them into the
            // reference's dL/dtransMat with this forward's records
            if (E.g16_moments) {
                if (E.gs3d)
                    mskern::launch_finish3d_grads(E.stream, E.n, P<float>(E.rec), P<float>(E.grads16));
                else
                    mskern::launch_finish_image_grads(E.stream, E.n, P<float>(E.rec), P<float>(E.grads16));
                E.g16_moments = false;
            }
            if (E.gs3d && which != MSPLAT_LAST_GRADS16) {
                set_err("buffer %d is a 2DGS raster gradient; the 3DGS mode's are in MSPLAT_LAST_GRADS16", which);
                return MSPLAT_E_ARG;
            }
            break;
        case MSPLAT_LAST_TRANSMATS: case MSPLAT_LAST_NORMALS:
            if (E.gs3d) {
                set_err("buffer %d does not exist in the 3DGS mode", which);
                return MSPLAT_E_ARG;
            }
            break;
        default: break;
    }
    const int64_t N = E.n, Pn = (int64_t)E.W * E.H;
    auto matf = [&](int idx, DevBuf &src, int stride, int off, int nf) -> int {
        CHECK(ensure(E.mat[idx], (size_t)N * nf * 4));
        mskern::launch_gather(E.stream, P<float>(src), stride, off, nf, P<float>(E.mat[idx]), (int)N);
        *ptr = E.mat[idx].p;
        *numel = N * nf;
        return MSPLAT_OK;
    };
    switch (which) {
        case MSPLAT_LAST_XYS: return E.gs3d ? matf(which, E.rec, 12, 0, 2) : matf(which, E.rec, 20, 9, 2);
        case MSPLAT_LAST_DEPTHS: *ptr = E.depths.p; *numel = N; return MSPLAT_OK;
        case MSPLAT_LAST_RADII: *ptr = E.radii.p; *numel = N; return MSPLAT_OK;
        case MSPLAT_LAST_NUM_TILES_HIT:
            CHECK(ensure(E.mat[which], (size_t)N * 4));
            mskern::launch_tiles_hit(E.stream, P<uint32_t>(E.rect), P<int>(E.radii), P<int>(E.mat[which]), (int)N);
            *ptr = E.mat[which].p;
            *numel = N;
            return MSPLAT_OK;
        case MSPLAT_LAST_TRANSMATS: return matf(which, E.rec, 20, 0, 9);
        case MSPLAT_LAST_COLORS_USED: return E.gs3d ? matf(which, E.rec, 12, 8, 3) : matf(which, E.rec, 20, 15, 3);
        case MSPLAT_LAST_OPACITY_SIGMOID:
            return E.gs3d ? matf(which, E.rec, 12, 5, 1) : matf(which, E.rec, 20, 11, 1);
        case MSPLAT_LAST_NORMALS: return matf(which, E.rec, 20, 12, 3);
        case MSPLAT_LAST_RECORDS: *ptr = E.rec.p; *numel = N * (E.gs3d ? mskern::kRec3Floats : 20); return MSPLAT_OK;
        case MSPLAT_LAST_TILE_OFFSETS:
            *ptr = E.offsets.p;
            *numel = (int64_t)E.tiles_x * E.tiles_y + 1;
            return MSPLAT_OK;
        case MSPLAT_LAST_GAUSSIAN_IDS: *ptr = E.ids.p; *numel = E.num_isect; return MSPLAT_OK;
        case MSPLAT_LAST_OUT_IMG: *ptr = E.out_img.p; *numel = Pn * 3; return MSPLAT_OK;
        case MSPLAT_LAST_FINAL_TS: *ptr = E.final_Ts.p; *numel = Pn * 3; return MSPLAT_OK;
        case MSPLAT_LAST_FINAL_IDX: *ptr = E.final_idx.p; *numel = Pn * 2; return MSPLAT_OK;
        case MSPLAT_LAST_OUT_DEPTH: *ptr = E.out_depth.p; *numel = Pn; return MSPLAT_OK;
        case MSPLAT_LAST_OUT_NORMAL: *ptr = E.out_normal.p; *numel = Pn * 3; return MSPLAT_OK;
        case MSPLAT_LAST_OUT_ALPHA: *ptr = E.out_alpha.p; *numel = Pn; return MSPLAT_OK;
        case MSPLAT_LAST_OUT_MEDIAN_DEPTH: *ptr = E.out_median.p; *numel = Pn; return MSPLAT_OK;
        case MSPLAT_LAST_OUT_DISTORTION: *ptr = E.out_dist.p; *numel = Pn; return MSPLAT_OK;
        case MSPLAT_LAST_DL_DOUT_IMG: *ptr = E.dL_dimg.p; *numel = E.dL_dimg.p ? Pn * 3 : 0; return MSPLAT_OK;
        case MSPLAT_LAST_GRADS16: *ptr = E.grads16.p; *numel = E.grads16.p ? N * 16 : 0; return MSPLAT_OK;
        case MSPLAT_LAST_DL_DTRANSMAT: return E.grads16.p ? matf(which, E.grads16, 16, 0, 9) : MSPLAT_OK;
        case MSPLAT_LAST_DL_DNORMAL3D: return E.grads16.p ? matf(which, E.grads16, 16, 9, 3) : MSPLAT_OK;
        case MSPLAT_LAST_DL_DOPACITY: return E.grads16.p ? matf(which, E.grads16, 16, 12, 1) : MSPLAT_OK;
        case MSPLAT_LAST_DL_DCOLORS: return E.grads16.p ? matf(which, E.grads16, 16, 13, 3) : MSPLAT_OK;
        case MSPLAT_LAST_DL_DMEAN3D: if (E.have_grads) { *ptr = E.dmeans.p; *numel = N * 3; } return MSPLAT_OK;
        case MSPLAT_LAST_DL_DSCALE:
            if (E.have_grads) {
                *ptr = E.dscales.p;
                *numel = N * (E.gs3d ? 3 : 2);
            }
            return MSPLAT_OK;
        case MSPLAT_LAST_DL_DQUAT: if (E.have_grads) { *ptr = E.dquats.p; *numel = N * 4; } return MSPLAT_OK;
        case MSPLAT_LAST_DL_DMEAN2D: if (E.have_grads) { *ptr = E.dmean2d.p; *numel = N * 2; } return MSPLAT_OK;
        case MSPLAT_LAST_DL_DFEATURES_DC: if (E.have_grads) { *ptr = E.dfdc.p; *numel = N * 3; } return MSPLAT_OK;
        case MSPLAT_LAST_DL_DFEATURES_REST:
            if (E.have_grads) { *ptr = E.dfrest.p; *numel = N * E.K3; }
            return MSPLAT_OK;
        case MSPLAT_LAST_BLEND_LOG:
            if (E.log_valid) { *ptr = E.blend_log.p; *numel = 64 * 4 * E.log_used; }
            return MSPLAT_OK;
        case MSPLAT_LAST_BLEND_CKPT:
            if (E.log_valid) { *ptr = E.t_ckpt.p; *numel = 64 * E.log_used; }
            return MSPLAT_OK;
        case MSPLAT_LAST_BLEND_CHUNKS:
            if (E.log_valid) {
                *ptr = E.log_table.p;
                *numel = (int64_t)msr::log_table_ints(E.num_isect, E.tiles_x * E.tiles_y);
            }
            return MSPLAT_OK;
        case MSPLAT_LAST_WAVE_COUNTS:
            if (E.log_valid) { *ptr = E.wave_cnt.p; *numel = 4 * (int64_t)E.tiles_x * E.tiles_y; }
            return MSPLAT_OK;
        default: set_err("unknown buffer id %d", which); return MSPLAT_E_ARG;
    }
}

}  // namespace

#define API_BEGIN                      \
    std::lock_guard<std::mutex> lk_(g_mu); \
    try {
#define API_END                                      \
    }                                                \
    catch (const std::exception &ex) {               \
        set_err("exception: %s", ex.what());         \
        return MSPLAT_E_ARG;                         \
    }                                                \
    catch (...) {                                    \
        set_err("unknown exception");                \
        return MSPLAT_E_ARG;                         \
    }

extern "C" {

int msplat_hip_init(void) {
    API_BEGIN
    return init_locked();
    API_END
}

void msplat_hip_cleanup(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    Engine &E = g_eng;
    if (!E.ready) return;
    (void)hipStreamSynchronize(E.stream);
    if (E.deep_stream) (void)hipStreamSynchronize(E.deep_stream);
    DevBuf *all[] = {&E.rec, &E.depths, &E.radii, &E.rect, &E.grads16, &E.colors_raw, &E.counts, &E.scan_tmp, &E.super_counts, &E.super_offsets, &E.super_cm, &E.super_tmp, &E.offsets,
                     &E.stats, &E.big_list, &E.huge_list, &E.chunk_base, &E.chunk_counts, &E.merge_base, &E.keys, &E.keys_tmp, &E.ids, &E.blend_log, &E.t_ckpt, &E.wave_cnt, &E.selfcheck, &E.out_img, &E.final_Ts,
                     &E.final_idx, &E.out_depth, &E.out_normal, &E.out_alpha, &E.out_median, &E.out_dist,
                     &E.dL_dimg, &E.gm1, &E.gs1, &E.gs12, &E.partials, &E.loss, &E.dmeans, &E.dscales,
                     &E.dquats, &E.dmean2d, &E.dfdc, &E.dfrest, &E.dens_flags, &E.dens_scan, &E.dens_keep, &E.dens_ws, &E.deep_list, &E.deep_pos, &E.deep_tb, &E.deep_cnt, &E.log_table, &E.log_ctr, &E.pair_counter,
                     &E.rgba, &E.tsdf_views, &E.tsdf_masks, &E.mc_cases, &E.chunk_cnt, &E.chunk_off};
    for (DevBuf *b : all) {
        if (b->p) (void)hipFree(b->p);
        *b = DevBuf{};
    }
    for (auto &b : E.mat) {
        if (b.p) (void)hipFree(b.p);
        b = DevBuf{};
    }
    E.dens_rows = 0;
    E.n_deep = 0;
    E.log_cap = 0;
    E.log_used = 0;
    E.log_fill[0] = E.log_fill[1] = 0.0;
    E.log_desc = msr::BlendLog{};
    E.n = 0;
    E.num_isect = 0;
    E.have_grads = false;
    E.raster_grads = false;
    E.g16_moments = false;
    E.log_valid = false;
    E.full_valid = false;
}

const char *msplat_hip_last_error(void) { return g_err; }

int msplat_hip_device_name(char *buf, int len) {
    API_BEGIN
    ENSURE_INIT();
    hipDeviceProp_t prop;
    HIPC(hipGetDeviceProperties(&prop, g_eng.device));
    snprintf(buf, (size_t)len, "%s (%s, %d CUs, %.0f GiB)", prop.name[0] ? prop.name : "AMD Instinct",
             prop.gcnArchName, prop.multiProcessorCount, (double)prop.totalGlobalMem / (1ull << 30));
    return MSPLAT_OK;
    API_END
}

void *msplat_hip_alloc(size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (init_locked() != MSPLAT_OK) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) {
        (void)hipGetLastError();
        set_err("hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int msplat_hip_free(void *p) {
    API_BEGIN
    if (!p) return MSPLAT_OK;
    ENSURE_INIT();
    HIPC(hipStreamSynchronize(g_eng.stream));
    HIPC(hipFree(p));
    return MSPLAT_OK;
    API_END
}

int msplat_hip_memset(void *p, int v, size_t bytes) {
    API_BEGIN
    ENSURE_INIT();
    HIPC(hipMemsetAsync(p, v, bytes, g_eng.stream));
    return MSPLAT_OK;
    API_END
}

int msplat_hip_upload(void *dst, const void *src, size_t bytes) {
    API_BEGIN
    ENSURE_INIT();
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_eng.stream));
    HIPC(hipStreamSynchronize(g_eng.stream));
    return MSPLAT_OK;
    API_END
}

// Device -> pageable host copy of `total` bytes through the two pinned
// chunks: the DMA of chunk k + 1 runs while the host moves chunk k on.
// Ordered after the work already on the engine stream; synchronous.
static int download_staged(unsigned char *dst, const unsigned char *src, size_t total) {
    Engine &E = g_eng;
    const size_t nch = (total + kD2HChunk - 1) / kD2HChunk;
    auto issue = [&](size_t k) -> int {
        const size_t off = k * kD2HChunk, len = std::min(kD2HChunk, total - off);
        HIPC(hipMemcpyAsync(E.stage + (k & 1) * kD2HChunk, src + off, len, hipMemcpyDeviceToHost, E.stream));
        HIPC(hipEventRecord(E.stage_ev[k & 1], E.stream));
        return MSPLAT_OK;
    };
    if (nch == 0) return MSPLAT_OK;
    CHECK(issue(0));
    if (nch > 1) CHECK(issue(1));
    for (size_t k = 0; k < nch; ++k) {
        HIPC(hipEventSynchronize(E.stage_ev[k & 1]));
        const size_t off = k * kD2HChunk, len = std::min(kD2HChunk, total - off);
        ms_parallel_memcpy(dst + off, E.stage + (k & 1) * kD2HChunk, len);
        if (k + 2 < nch) CHECK(issue(k + 2));
    }
    return MSPLAT_OK;
}

int msplat_hip_download(void *dst, const void *src, size_t bytes) {
    API_BEGIN
    ENSURE_INIT();
    if (bytes >= kD2HChunk)  // large: staged (pageable destinations copy ~3x faster)
        return download_staged(static_cast<unsigned char *>(dst), static_cast<const unsigned char *>(src), bytes);
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_eng.stream));
    HIPC(hipStreamSynchronize(g_eng.stream));
    return MSPLAT_OK;
    API_END
}

int msplat_hip_copy(void *dst, const void *src, size_t bytes) {
    API_BEGIN
    ENSURE_INIT();
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_eng.stream));
    return MSPLAT_OK;
    API_END
}

int msplat_hip_commit(void) { return MSPLAT_OK; }

int msplat_hip_sync(void) {
    API_BEGIN
    ENSURE_INIT();
    HIPC(hipStreamSynchronize(g_eng.stream));
    return MSPLAT_OK;
    API_END
}

int msplat_hip_image_to_rgba8(const float *img, int64_t num_pixels, uint8_t *rgba_host) {
    API_BEGIN
    ENSURE_INIT();
    if (num_pixels < 0 || (num_pixels > 0 && (!img || !rgba_host))) {
        set_err("invalid rgba8 arguments");
        return MSPLAT_E_ARG;
    }
    if (num_pixels == 0) return MSPLAT_OK;
    Engine &E = g_eng;
    CHECK(ensure(E.rgba, (size_t)num_pixels * 4));
    mskern::launch_rgba8(E.stream, img, num_pixels, P<uint32_t>(E.rgba));
    HIPC(hipGetLastError());
    return download_staged(rgba_host, P<unsigned char>(E.rgba), (size_t)num_pixels * 4);
    API_END
}

// ---- mesh extraction ------------------------------------------------------

int msplat_hip_mc_table(int8_t tri[256 * 16]) {
    if (!tri) {
        set_err("null table");
        return MSPLAT_E_ARG;
    }
    mskern::mc_table_host(tri);
    return MSPLAT_OK;
}

namespace {
bool grid_args_ok(const float *grid, int dx, int dy, int dz, const float origin[3]) {
    // (the TSDF launch needs its 8 x 8 x 4 bricks, padded to 8, in an int)
    if (!grid || !origin || dx < 1 || dy < 1 || dz < 1 || dz > 65535 ||
        (uint64_t)dx * (uint64_t)dy >= (uint64_t(1) << 32) ||
        (int64_t)((dx + 7) / 8) * ((dy + 7) / 8) * ((dz + 3) / 4) > (int64_t)INT_MAX - 8) {
        set_err("invalid voxel grid (%d x %d x %d)", dx, dy, dz);
        return false;
    }
    return true;
}
}  // namespace

int msplat_hip_tsdf_integrate(float *grid, int dx, int dy, int dz, const float origin[3], float voxel_size,
                              const MsplatTsdfView *views, int num_views, float trunc_dist, float alpha_thresh) {
    API_BEGIN
    ENSURE_INIT();
    if (!grid_args_ok(grid, dx, dy, dz, origin)) return MSPLAT_E_ARG;
    if (num_views < 0 || (num_views > 0 && !views)) {
        set_err("invalid TSDF views");
        return MSPLAT_E_ARG;
    }
    for (int k = 0; k < num_views; ++k)
        if (views[k].width < 1 || views[k].height < 1 || !views[k].depth_dev || !views[k].alpha_dev) {
            set_err("TSDF view %d: empty map or null pointer", k);
            return MSPLAT_E_ARG;
        }
    if (num_views == 0) return MSPLAT_OK;
    Engine &E = g_eng;
    // each view's pass mask, then the fold
    std::vector<mskern::TsdfViewDev> dv((size_t)num_views);
    size_t words = 0;
    int64_t max_segs = 0;
    for (int k = 0; k < num_views; ++k) {
        dv[k].v = views[k];
        dv[k].words_per_row = mskern::tsdf_mask_words(views[k].width);
        words += (size_t)dv[k].words_per_row * views[k].height;
        max_segs = std::max<int64_t>(max_segs, (int64_t)((views[k].width + 63) / 64) * views[k].height);
    }
    if (max_segs > (int64_t)INT_MAX) {
        set_err("TSDF view too large");
        return MSPLAT_E_ARG;
    }
    CHECK(ensure(E.tsdf_masks, words * 4));
    size_t off = 0;
    for (auto &d : dv) {
        d.mask = P<uint32_t>(E.tsdf_masks) + off;
        off += (size_t)d.words_per_row * d.v.height;
    }
    const size_t bytes = dv.size() * sizeof(mskern::TsdfViewDev);
    CHECK(ensure(E.tsdf_views, bytes));
    HIPC(hipMemcpyAsync(E.tsdf_views.p, dv.data(), bytes, hipMemcpyHostToDevice, E.stream));
    const auto *vdev = P<mskern::TsdfViewDev>(E.tsdf_views);
    mskern::launch_tsdf_masks(E.stream, vdev, num_views, max_segs, alpha_thresh);
    mskern::launch_tsdf_integrate(E.stream, grid, dx, dy, dz, origin, voxel_size, vdev, num_views, trunc_dist);
    HIPC(hipGetLastError());
    // the view records are rewritten by the next call
    HIPC(hipStreamSynchronize(E.stream));
    return MSPLAT_OK;
    API_END
}

int msplat_hip_marching_cubes(const float *grid, int dx, int dy, int dz, const float origin[3], float voxel_size,
                              int64_t max_triangles, float *tris, int64_t *num_triangles, int64_t *num_emitted) {
    API_BEGIN
    ENSURE_INIT();
    if (!grid_args_ok(grid, dx, dy, dz, origin)) return MSPLAT_E_ARG;
    if (!num_triangles || max_triangles < 0 || (max_triangles > 0 && !tris)) {
        set_err("invalid marching-cubes output");
        return MSPLAT_E_ARG;
    }
    *num_triangles = 0;
    if (num_emitted) *num_emitted = 0;
    const int64_t nc = mskern::mc_num_cells(dx, dy, dz);
    if (nc == 0) return MSPLAT_OK;
    const int64_t nch = mskern::mesh_chunks(nc);
    if (nch > (int64_t)INT_MAX) {
        set_err("voxel grid too large");
        return MSPLAT_E_ARG;
    }
    Engine &E = g_eng;
    hipStream_t s = E.stream;
    CHECK(ensure(E.mc_cases, (size_t)nch * mskern::kMeshChunk));
    CHECK(ensure(E.chunk_cnt, (size_t)nch * 4));
    CHECK(ensure(E.chunk_off, (size_t)(nch + 1) * 8));
    mskern::launch_mc_classify(s, grid, dx, dy, dz, P<uint8_t>(E.mc_cases), P<uint32_t>(E.chunk_cnt));
    mskern::launch_chunk_scan(s, P<uint32_t>(E.chunk_cnt), nch, P<uint64_t>(E.chunk_off));
    if (max_triangles > 0)
        mskern::launch_mc_emit(s, grid, dx, dy, dz, origin, voxel_size, P<uint8_t>(E.mc_cases),
                               P<uint64_t>(E.chunk_off), max_triangles, tris);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(E.pinned_d, P<uint64_t>(E.chunk_off) + nch, 8, hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
    uint64_t total;
    std::memcpy(&total, E.pinned_d, 8);
    *num_triangles = std::min<int64_t>((int64_t)total, max_triangles);
    if (num_emitted) *num_emitted = (int64_t)total;
    return MSPLAT_OK;
    API_END
}

int msplat_hip_unproject_depth(const float *img, const float *depth, const float *alpha, int width, int height,
                               float fx, float fy, float cx, float cy, const float cam_to_world[16],
                               float alpha_thresh, float *xyz, uint8_t *rgb, int64_t *num_points) {
    API_BEGIN
    ENSURE_INIT();
    if (!num_points || !cam_to_world || width < 0 || height < 0 ||
        ((int64_t)width * height > 0 && (!img || !depth || !alpha || !xyz || !rgb))) {
        set_err("invalid unprojection arguments");
        return MSPLAT_E_ARG;
    }
    *num_points = 0;
    const int64_t np = (int64_t)width * height;
    if (np == 0) return MSPLAT_OK;
    const int64_t nch = mskern::mesh_chunks(np);
    Engine &E = g_eng;
    hipStream_t s = E.stream;
    CHECK(ensure(E.chunk_cnt, (size_t)nch * 4));
    CHECK(ensure(E.chunk_off, (size_t)(nch + 1) * 8));
    mskern::launch_unproject_count(s, img, depth, alpha, width, height, fx, fy, cx, cy, cam_to_world, alpha_thresh,
                                   P<uint32_t>(E.chunk_cnt));
    mskern::launch_chunk_scan(s, P<uint32_t>(E.chunk_cnt), nch, P<uint64_t>(E.chunk_off));
    mskern::launch_unproject_emit(s, img, depth, alpha, width, height, fx, fy, cx, cy, cam_to_world, alpha_thresh,
                                  P<uint64_t>(E.chunk_off), xyz, rgb);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(E.pinned_d, P<uint64_t>(E.chunk_off) + nch, 8, hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
    uint64_t total;
    std::memcpy(&total, E.pinned_d, 8);
    *num_points = (int64_t)total;
    return MSPLAT_OK;
    API_END
}

int msplat_hip_render(const MsplatCamera *cam, const MsplatGaussians *g, const float *bg, int64_t *nisect) {
    API_BEGIN
    ENSURE_INIT();
    CHECK(forward_locked(cam, g, bg, nisect, false, false));
    stage_mark(ST_LOSS);
    if (g_eng.count_pairs) {
        HIPC(hipMemcpyAsync(g_eng.pairs, g_eng.pair_counter.p, 40, hipMemcpyDeviceToHost, g_eng.stream));
        HIPC(hipStreamSynchronize(g_eng.stream));
    }
    if (g_eng.timing) {
        HIPC(hipStreamSynchronize(g_eng.stream));
        for (int i = ST_PROJECT; i < ST_LOSS; ++i) {
            HIPC(hipEventElapsedTime(&g_eng.stage_ms[i], g_eng.ev[i], g_eng.ev[i + 1]));
            g_eng.stage_valid[i] = true;
        }
    }
    return MSPLAT_OK;
    API_END
}

static int train_step_once(const MsplatCamera *cam, const MsplatGaussians *g, const float *bg, const float *gt,
                          float lambda_l1, float lambda_dist, float lambda_dssim, float *gnorm, float *vis,
                          float *max2d, float inv_max_dim, const MsplatAdam *adam, float *loss_host,
                          int64_t *nisect, bool *log_overflow) {
    if (!gt || !gnorm || !vis || !max2d) {
        set_err("null gt / densify statistics");
        return MSPLAT_E_ARG;
    }
    Engine &E = g_eng;
    hipStream_t s = E.stream;
    // the deep tiles' log rebuild runs beside the loss (the raster
    // backward's deep part follows it on the deep-tile stream)
    E.defer_deep_log = true;
    const int fr = forward_locked(cam, g, bg, nisect, true, lambda_dist != 0.f);
    E.defer_deep_log = false;
    CHECK(fr);
    const int N = g->num_points, W = cam->width, H = cam->height;
    const size_t Pn = (size_t)W * H;
    stage_mark(ST_LOSS);
    CHECK(ensure(E.dL_dimg, Pn * 12));
    CHECK(loss_locked(W, H, P<float>(E.out_img), gt, lambda_dist != 0.f ? P<float>(E.out_dist) : nullptr,
                      lambda_l1, lambda_dist, lambda_dssim, P<float>(E.dL_dimg)));
    HIPC(hipMemcpyAsync(E.pinned_d, E.loss.p, 2 * sizeof(double), hipMemcpyDeviceToHost, s));
    stage_mark(ST_RASTER_BWD);
    CHECK(ensure(E.grads16, (size_t)N * 64));
    mskern::launch_zero16(s, P<float>(E.grads16), (int64_t)N * 4);
    const float inv_np = 1.0f / (float)((unsigned)H * (unsigned)W * 3u);
    const float ddist_uniform = lambda_dist * (inv_np * 3.0f);
    mskern::DeepTiles deep;
    CHECK(deep_tiles(deep));
    // the layout the logging forward planned (a new plan could reallocate
    // the pool under the log)
    const msr::BlendLog blog = E.log_desc;
    const bool t_moments = mskern::launch_raster_bwd(s, W, H, cam->tiles_x, cam->tiles_y, P<int>(E.offsets), blog,
                              P<float>(E.rec), bg, P<float>(E.final_Ts),
                              P<int>(E.final_idx), P<float>(E.dL_dimg), nullptr, nullptr, nullptr, nullptr, nullptr,
                              ddist_uniform, P<float>(E.grads16), deep);
    stage_mark(ST_PROJECT_BWD);
    if (adam) {
        mskern::launch_project_bwd(s, *cam, *g, P<int>(E.radii), P<float>(E.grads16), nullptr, nullptr, nullptr,
                                   nullptr, nullptr, nullptr, gnorm, vis, max2d, inv_max_dim, adam,
                                   t_moments ? P<float>(E.rec) : nullptr, blog.overflow, 0);
    } else {
        CHECK(ensure(E.dmeans, (size_t)N * 12));
        CHECK(ensure(E.dscales, (size_t)N * 8));
        CHECK(ensure(E.dquats, (size_t)N * 16));
        CHECK(ensure(E.dmean2d, (size_t)N * 8));
        CHECK(ensure(E.dfdc, (size_t)N * 12));
        CHECK(ensure(E.dfrest, (size_t)N * E.K3 * 4));
        mskern::launch_project_bwd(s, *cam, *g, P<int>(E.radii), P<float>(E.grads16), P<float>(E.dmeans),
                                   P<float>(E.dscales), P<float>(E.dquats), P<float>(E.dmean2d), P<float>(E.dfdc),
                                   P<float>(E.dfrest), gnorm, vis, max2d, inv_max_dim, nullptr,
                                   t_moments ? P<float>(E.rec) : nullptr, blog.overflow, 0);
        E.have_grads = true;
    }
    E.raster_grads = true;
    E.g16_moments = t_moments;
    stage_mark(ST_COUNT);
    CHECK(log_readback(blog, s));
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(s));
    *log_overflow = log_account(blog);
    if (*log_overflow) {
        E.have_grads = E.raster_grads = false;
        return MSPLAT_OK;
    }
    if (loss_host) *loss_host = (float)E.pinned_d[0];
    if (E.count_pairs) {
        HIPC(hipMemcpyAsync(E.pairs, E.pair_counter.p, 40, hipMemcpyDeviceToHost, s));
        HIPC(hipStreamSynchronize(s));
    }
    if (E.timing) {
        for (int i = 0; i < ST_COUNT; ++i) {
            HIPC(hipEventElapsedTime(&E.stage_ms[i], E.ev[i], E.ev[i + 1]));
            E.stage_valid[i] = true;
        }
    }
    return MSPLAT_OK;
}

int msplat_hip_train_step(const MsplatCamera *cam, const MsplatGaussians *g, const float *bg, const float *gt,
                          float lambda_l1, float lambda_dist, float lambda_dssim, float *gnorm, float *vis,
                          float *max2d, float inv_max_dim, const MsplatAdam *adam, float *loss_host,
                          int64_t *nisect) {
    API_BEGIN
    ENSURE_INIT();
    // a step whose blend log overflowed the pool changed nothing (its
    // backward and Adam skip): redo it with a larger pool
    for (;;) {
        bool overflow = false;
        CHECK(train_step_once(cam, g, bg, gt, lambda_l1, lambda_dist, lambda_dssim, gnorm, vis, max2d, inv_max_dim, adam, loss_host, nisect, &overflow));
        if (!overflow) return MSPLAT_OK;
        grow_log_pool();
    }
    API_END
}

// ---- 3DGS mode ----------------------------------------------------------

int msplat_hip_render_3dgs(const MsplatCamera *cam, const MsplatGaussians *g, const float *bg, int64_t *nisect) {
    API_BEGIN
    ENSURE_INIT();
    CHECK(forward_locked(cam, g, bg, nisect, false, false, true));
    stage_mark(ST_LOSS);
    if (g_eng.timing) {
        HIPC(hipStreamSynchronize(g_eng.stream));
        for (int i = ST_PROJECT; i < ST_LOSS; ++i) {
            HIPC(hipEventElapsedTime(&g_eng.stage_ms[i], g_eng.ev[i], g_eng.ev[i + 1]));
            g_eng.stage_valid[i] = true;
        }
    }
    return MSPLAT_OK;
    API_END
}

static int train_step3d_once(const MsplatCamera *cam, const MsplatGaussians *g, const float *bg, const float *gt,
                               float lambda_l1, float lambda_dssim, float *gnorm, float *vis, float *max2d,
                               float inv_max_dim, const MsplatAdam *adam, float *loss_host, int64_t *nisect,
                               bool *log_overflow) {
    if (!gt || !gnorm || !vis || !max2d) {
        set_err("null gt / densify statistics");
        return MSPLAT_E_ARG;
    }
    Engine &E = g_eng;
    hipStream_t s = E.stream;
    CHECK(forward_locked(cam, g, bg, nisect, true, false, true));
    const int N = g->num_points, W = cam->width, H = cam->height;
    const size_t Pn = (size_t)W * H;
    stage_mark(ST_LOSS);
    CHECK(ensure(E.dL_dimg, Pn * 12));
    CHECK(loss_locked(W, H, P<float>(E.out_img), gt, nullptr, lambda_l1, 0.f, lambda_dssim, P<float>(E.dL_dimg)));
    HIPC(hipMemcpyAsync(E.pinned_d, E.loss.p, 2 * sizeof(double), hipMemcpyDeviceToHost, s));
    stage_mark(ST_RASTER_BWD);
    CHECK(ensure(E.grads16, (size_t)N * 64));
    mskern::launch_zero16(s, P<float>(E.grads16), (int64_t)N * 4);
    // the layout the logging forward planned (a new plan could reallocate
    // the pool under the log)
    const msr::BlendLog blog = E.log_desc;
    mskern::launch_raster3d_bwd(s, W, H, cam->tiles_x, cam->tiles_y, P<int>(E.offsets), blog, P<float>(E.rec), bg,
                                P<float>(E.final_Ts), P<float>(E.dL_dimg), P<float>(E.grads16));
    stage_mark(ST_PROJECT_BWD);
    if (adam) {
        mskern::launch_project3d_bwd(s, *cam, *g, P<int>(E.radii), P<float>(E.grads16), nullptr, nullptr, nullptr,
                                     nullptr, nullptr, nullptr, gnorm, vis, max2d, inv_max_dim, adam,
                                     P<float>(E.rec), blog.overflow, 0);
    } else {
        CHECK(ensure(E.dmeans, (size_t)N * 12));
        CHECK(ensure(E.dscales, (size_t)N * 12));
        CHECK(ensure(E.dquats, (size_t)N * 16));
        CHECK(ensure(E.dmean2d, (size_t)N * 8));
        CHECK(ensure(E.dfdc, (size_t)N * 12));
        CHECK(ensure(E.dfrest, (size_t)N * E.K3 * 4));
        mskern::launch_project3d_bwd(s, *cam, *g, P<int>(E.radii), P<float>(E.grads16), P<float>(E.dmeans),
                                     P<float>(E.dscales), P<float>(E.dquats), P<float>(E.dmean2d),
                                     P<float>(E.dfdc), P<float>(E.dfrest), gnorm, vis, max2d, inv_max_dim, nullptr,
                                     P<float>(E.rec), blog.overflow, 0);
        E.have_grads = true;
    }
    E.raster_grads = true;
    E.g16_moments = true;
    stage_mark(ST_COUNT);
    CHECK(log_readback(blog, s));
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(s));
    *log_overflow = log_account(blog);
    if (*log_overflow) {
        E.have_grads = E.raster_grads = false;
        return MSPLAT_OK;
    }
    if (loss_host) *loss_host = (float)E.pinned_d[0];
    if (E.timing) {
        for (int i = 0; i < ST_COUNT; ++i) {
            HIPC(hipEventElapsedTime(&E.stage_ms[i], E.ev[i], E.ev[i + 1]));
            E.stage_valid[i] = true;
        }
    }
    return MSPLAT_OK;
}

int msplat_hip_train_step_3dgs(const MsplatCamera *cam, const MsplatGaussians *g, const float *bg, const float *gt,
                               float lambda_l1, float lambda_dssim, float *gnorm, float *vis, float *max2d,
                               float inv_max_dim, const MsplatAdam *adam, float *loss_host, int64_t *nisect) {
    API_BEGIN
    ENSURE_INIT();
    // a step whose blend log overflowed the pool changed nothing (its
    // backward and Adam skip): redo it with a larger pool
    for (;;) {
        bool overflow = false;
        CHECK(train_step3d_once(cam, g, bg, gt, lambda_l1, lambda_dssim, gnorm, vis, max2d, inv_max_dim, adam, loss_host, nisect, &overflow));
        if (!overflow) return MSPLAT_OK;
        grow_log_pool();
    }
    API_END
}

int msplat_hip_fused_adam(float *p, const float *gr, float *m, float *v, int64_t n, float step, float b1, float b2,
                          float bc2_sqrt, float eps) {
    API_BEGIN
    ENSURE_INIT();
    if (n < 0 || (n > 0 && (!p || !gr || !m || !v))) {
        set_err("invalid adam arguments");
        return MSPLAT_E_ARG;
    }
    mskern::launch_adam(g_eng.stream, p, gr, m, v, n, step, b1, b2, bc2_sqrt, eps);
    HIPC(hipGetLastError());
    return MSPLAT_OK;
    API_END
}

static int densify_impl(int scale_dim, int n, int capacity, float grad_thresh, float size_thresh,
                        float screen_thresh, int check_screen, float cull_alpha_thresh, float cull_scale_thresh,
                        float cull_screen_size, int check_huge, const float *gnorm, const float *vis,
                        const float *max2d, float half_max_dim, float *const params[6], int fr_stride,
                        float *const exp_avg[6], float *const exp_avg_sq[6], const float *random, int *new_count) {
    if (n < 0 || n > capacity || fr_stride < 0 || !new_count || !gnorm || !vis || !max2d || !random) {
        set_err("densify: N (%d) exceeds capacity %d or bad arguments", n, capacity);
        return MSPLAT_E_ARG;
    }
    if (n == 0) {
        *new_count = 0;
        return MSPLAT_OK;
    }
    Engine &E = g_eng;
    const int strides[6] = {3, scale_dim, 4, 3, fr_stride, 1};
    mskern::DensifyArgs a{};
    a.n = n;
    a.fr_stride = fr_stride;
    a.scale_dim = scale_dim;
    a.grad_th = grad_thresh;
    a.size_th = size_thresh;
    a.screen_th = screen_thresh;
    a.check_screen = check_screen;
    a.cull_alpha = cull_alpha_thresh;
    a.cull_scale = cull_scale_thresh;
    a.cull_screen = cull_screen_size;
    a.check_huge = check_huge;
    a.grad_norm = gnorm;
    a.vis = vis;
    a.max2d = max2d;
    a.half_max_dim = half_max_dim;
    a.log_size_fac = std::log(1.6f);
    a.random = random;
    for (int gi = 0; gi < 6; ++gi) {
        a.params[gi] = params[gi];
        a.exp_avg[gi] = exp_avg[gi];
        a.exp_avg_sq[gi] = exp_avg_sq[gi];
    }
    // four int flags per splat; regrown to twice the splat count (at most
    // the capacity) when it no longer fits
    if (E.dens_flags.cap < (size_t)n * 16)
        CHECK(ensure(E.dens_flags, (size_t)std::min<int64_t>(2 * (int64_t)n, capacity) * 16));
    // the count after appending is at most 4N (a splat can be split and dup)
    CHECK(ensure(E.dens_scan, (size_t)mskern::scan_temp_ints(4 * (int64_t)n) * 4));
    int *f = P<int>(E.dens_flags);
    a.split = f;
    a.dup = f + n;
    a.split_pre = f + 2 * (size_t)n;
    a.dup_pre = f + 3 * (size_t)n;
    a.scan_temp = P<int>(E.dens_scan);
    mskern::launch_densify_classify(E.stream, a);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(E.pinned_i, a.split_pre + n - 1, sizeof(int), hipMemcpyDeviceToHost, E.stream));
    HIPC(hipMemcpyAsync(E.pinned_i + 1, a.dup_pre + n - 1, sizeof(int), hipMemcpyDeviceToHost, E.stream));
    HIPC(hipStreamSynchronize(E.stream));
    // A splat that is small but wide on screen is classified both split and
    // dup (msplat_metal.metal:3250-3262), so the appended count can exceed
    // the reference's 3N worst case (msplat_metal.mm:1358, where the dup
    // writes then run past the buffers).  Nothing has been written yet:
    // refuse and report the rows needed, so the caller can grow and retry.
    const int64_t n_new = (int64_t)n + 2 * (int64_t)E.pinned_i[0] + E.pinned_i[1];
    if (n_new > capacity) {
        *new_count = n_new > INT32_MAX ? INT32_MAX : (int)n_new;
        set_err("densify: %lld rows needed after appending, capacity is %d", (long long)n_new, capacity);
        return MSPLAT_E_CAPACITY;
    }
    for (int gi = 0; gi < 6; ++gi)
        if (strides[gi] > 127) {
            set_err("densify: row stride %d above 127 floats", strides[gi]);
            return MSPLAT_E_ARG;
        }
    // Workspace and row maps are sized for the caller's capacity (the bound
    // on the rows after appending), so they are allocated once per capacity
    // instead of once per cycle of a model that doubles every cycle.
    const int64_t rows = capacity;
    if (n_new > E.dens_rows) {
        CHECK(ensure(E.dens_ws, (size_t)mskern::densify_workspace_floats((int)rows, scale_dim, fr_stride) * 4));
        CHECK(ensure(E.dens_keep, (size_t)rows * 4 * 4));
        E.dens_rows = rows;
    } else {
        CHECK(ensure(E.dens_ws, (size_t)mskern::densify_workspace_floats((int)n_new, scale_dim, fr_stride) * 4));
    }
    a.workspace = P<float>(E.dens_ws);
    a.keep = P<int>(E.dens_keep);
    a.keep_pre = a.keep + n_new;
    a.src_of = a.keep + 2 * n_new;
    a.parent = a.keep + 3 * n_new;
    mskern::launch_densify_apply(E.stream, a, E.pinned_i[0], (int)n_new);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(E.pinned_i, a.keep_pre + n_new - 1, sizeof(int), hipMemcpyDeviceToHost, E.stream));
    HIPC(hipStreamSynchronize(E.stream));
    *new_count = E.pinned_i[0];
    return MSPLAT_OK;
}

int msplat_hip_densify(int n, int capacity, float grad_thresh, float size_thresh, float screen_thresh,
                       int check_screen, float cull_alpha_thresh, float cull_scale_thresh, float cull_screen_size,
                       int check_huge, const float *gnorm, const float *vis, const float *max2d, float half_max_dim,
                       float *const params[6], int fr_stride, float *const exp_avg[6], float *const exp_avg_sq[6],
                       const float *random, int *new_count) {
    API_BEGIN
    ENSURE_INIT();
    return densify_impl(2, n, capacity, grad_thresh, size_thresh, screen_thresh, check_screen, cull_alpha_thresh,
                        cull_scale_thresh, cull_screen_size, check_huge, gnorm, vis, max2d, half_max_dim, params,
                        fr_stride, exp_avg, exp_avg_sq, random, new_count);
    API_END
}

int msplat_hip_densify_3dgs(int n, int capacity, float grad_thresh, float size_thresh, float screen_thresh,
                            int check_screen, float cull_alpha_thresh, float cull_scale_thresh,
                            float cull_screen_size, int check_huge, const float *gnorm, const float *vis,
                            const float *max2d, float half_max_dim, float *const params[6], int fr_stride,
                            float *const exp_avg[6], float *const exp_avg_sq[6], const float *random,
                            int *new_count) {
    API_BEGIN
    ENSURE_INIT();
    return densify_impl(3, n, capacity, grad_thresh, size_thresh, screen_thresh, check_screen, cull_alpha_thresh,
                        cull_scale_thresh, cull_screen_size, check_huge, gnorm, vis, max2d, half_max_dim, params,
                        fr_stride, exp_avg, exp_avg_sq, random, new_count);
    API_END
}

int msplat_hip_clamp_max(float *p, int64_t n, float value) {
    API_BEGIN
    ENSURE_INIT();
    if (n < 0 || (n > 0 && !p)) {
        set_err("invalid clamp arguments");
        return MSPLAT_E_ARG;
    }
    mskern::launch_clamp_max(g_eng.stream, p, n, value);
    HIPC(hipGetLastError());
    return MSPLAT_OK;
    API_END
}

int msplat_hip_loss_fwd_bwd(int W, int H, const float *img, const float *gt, const float *dist, float l1,
                            float ldist, float ldssim, float *dL, double *loss_host, double *ssim_host) {
    API_BEGIN
    ENSURE_INIT();
    if (W <= 0 || H <= 0 || !img || !gt || !dL || (ldist != 0.f && !dist)) {
        set_err("invalid loss arguments");
        return MSPLAT_E_ARG;
    }
    CHECK(loss_locked(W, H, img, gt, ldist != 0.f ? dist : nullptr, l1, ldist, ldssim, dL));
    HIPC(hipMemcpyAsync(g_eng.pinned_d, g_eng.loss.p, 2 * sizeof(double), hipMemcpyDeviceToHost, g_eng.stream));
    HIPC(hipStreamSynchronize(g_eng.stream));
    if (loss_host) *loss_host = g_eng.pinned_d[0];
    if (ssim_host) *ssim_host = g_eng.pinned_d[1];
    return MSPLAT_OK;
    API_END
}

int msplat_hip_loss_fwd_bwd_noalloc(int W, int H, const float *img, const float *gt, const float *dist, float l1,
                                    float ldist, float ldssim, float *dL, double *loss_host, double *ssim_host) {
    API_BEGIN
    // no set-up here: msplat_hip_init allocated the stream and the pinned
    // readback area and looked up this device's scratch array
    if (!g_eng.ready) {
        set_err("loss_fwd_bwd_noalloc: call msplat_hip_init first (this entry point allocates nothing)");
        return MSPLAT_E_ARG;
    }
    if (W <= 0 || H <= 0 || !img || !gt || !dL || (ldist != 0.f && !dist)) {
        set_err("invalid loss arguments");
        return MSPLAT_E_ARG;
    }
    const int64_t pixels = (int64_t)W * H;
    if (pixels > kNoAllocMaxPixels) {
        set_err("loss_fwd_bwd_noalloc: %dx%d = %lld pixels exceeds the %lld-pixel scratch", W, H,
                (long long)pixels, (long long)kNoAllocMaxPixels);
        return MSPLAT_E_CAPACITY;
    }
    if ((int64_t)mskern::loss_num_partials(W, H) > kNoAllocMaxBlocks) {
        set_err("loss_fwd_bwd_noalloc: %dx%d needs more than %lld tiles", W, H, (long long)kNoAllocMaxBlocks);
        return MSPLAT_E_CAPACITY;
    }
    Engine &E = g_eng;
    unsigned char *base = static_cast<unsigned char *>(g_scratch_dev[E.device]);
    if (!base) {
        set_err("loss_fwd_bwd_noalloc: no scratch address for device %d", E.device);
        return MSPLAT_E_HIP;
    }
    float *gm1 = reinterpret_cast<float *>(base);
    float *gs1 = reinterpret_cast<float *>(base + kNoAllocMapBytes);
    float *gs12 = reinterpret_cast<float *>(base + 2 * kNoAllocMapBytes);
    double *partials = reinterpret_cast<double *>(base + kNoAllocPartialsOff);
    double *loss = reinterpret_cast<double *>(base + kNoAllocLossOff);
    mskern::launch_loss_fwd_bwd(E.stream, W, H, img, gt, ldist != 0.f ? dist : nullptr, l1, ldist, ldssim, E.window,
                                gm1, gs1, gs12, partials, loss, dL);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(E.pinned_d, loss, 2 * sizeof(double), hipMemcpyDeviceToHost, E.stream));
    HIPC(hipStreamSynchronize(E.stream));
    if (loss_host) *loss_host = E.pinned_d[0];
    if (ssim_host) *ssim_host = E.pinned_d[1];
    return MSPLAT_OK;
    API_END
}

int msplat_hip_raster_bwd(const float *dL_dimg, const float *dL_ddepth, const float *dL_dalpha,
                          const float *dL_dnormal, const float *dL_dmedian, const float *dL_ddist, float *grads16) {
    API_BEGIN
    ENSURE_INIT();
    Engine &E = g_eng;
    if (!E.rec.p || !E.bg || !dL_dimg || !grads16) {
        set_err("raster_bwd needs a preceding forward and dL_dimg / grads16");
        return MSPLAT_E_ARG;
    }
    if (E.gs3d) {
        set_err("raster_bwd is the 2DGS backward; the 3DGS mode's runs inside msplat_hip_train_step_3dgs");
        return MSPLAT_E_ARG;
    }
    // a render-only forward skips the blend log, a training forward the full
    // outputs; replay the deterministic raster forward with what is missing
    const bool need_full = dL_ddepth || dL_dalpha || dL_dnormal || dL_dmedian || dL_ddist;
    if (!E.log_valid || (need_full && !E.full_valid)) CHECK(log_forward_checked(need_full || E.full_valid));
    mskern::DeepTiles deep;
    CHECK(deep_tiles(deep));
    // the layout the logging forward planned (a new plan could reallocate
    // the pool under the log)
    const msr::BlendLog blog = E.log_desc;
    const bool t_moments = mskern::launch_raster_bwd(
        E.stream, E.W, E.H, E.tiles_x, E.tiles_y, P<int>(E.offsets), blog, P<float>(E.rec), E.bg,
        P<float>(E.final_Ts), P<int>(E.final_idx), dL_dimg, dL_ddepth, dL_dalpha, dL_dnormal, dL_dmedian, dL_ddist,
        0.0f, grads16, deep);
    if (t_moments) mskern::launch_finish_image_grads(E.stream, E.n, P<float>(E.rec), grads16);
    HIPC(hipGetLastError());
    return MSPLAT_OK;
    API_END
}

int msplat_hip_project_bwd(const MsplatCamera *cam, const MsplatGaussians *g, const int32_t *radii,
                           const float *g16, float *dmeans, float *dscales, float *dquats, float *dmean2d,
                           float *dfdc, float *dfrest, float *gnorm, float *vis, float *max2d, float inv_max_dim) {
    API_BEGIN
    ENSURE_INIT();
    CHECK(validate_cam(cam, g));
    if (!radii || !g16 || !dmeans || !dscales || !dquats || !dmean2d || !dfdc || (cam->degree > 0 && !dfrest) ||
        !gnorm || !vis || !max2d) {
        set_err("invalid project_bwd arguments");
        return MSPLAT_E_ARG;
    }
    mskern::launch_project_bwd(g_eng.stream, *cam, *g, radii, g16, dmeans, dscales, dquats, dmean2d, dfdc, dfrest,
                               gnorm, vis, max2d, inv_max_dim, nullptr, nullptr);
    HIPC(hipGetLastError());
    return MSPLAT_OK;
    API_END
}

int msplat_hip_project_bwd_adam(const MsplatCamera *cam, const MsplatGaussians *g, const int32_t *radii,
                                const float *g16, float *gnorm, float *vis, float *max2d, float inv_max_dim,
                                const MsplatAdam *adam) {
    API_BEGIN
    ENSURE_INIT();
    CHECK(validate_cam(cam, g));
    if (!radii || !g16 || !gnorm || !vis || !max2d || !adam) {
        set_err("invalid project_bwd_adam arguments");
        return MSPLAT_E_ARG;
    }
    mskern::launch_project_bwd(g_eng.stream, *cam, *g, radii, g16, nullptr, nullptr, nullptr, nullptr, nullptr,
                               nullptr, gnorm, vis, max2d, inv_max_dim, adam, nullptr);
    HIPC(hipGetLastError());
    return MSPLAT_OK;
    API_END
}

int msplat_hip_last(int which, void **ptr, int64_t *numel) {
    API_BEGIN
    ENSURE_INIT();
    if (!ptr || !numel) return MSPLAT_E_ARG;
    CHECK(last_locked(which, ptr, numel));
    HIPC(hipGetLastError());
    return MSPLAT_OK;
    API_END
}

int msplat_hip_enable_timing(int enable) {
    API_BEGIN
    ENSURE_INIT();
    g_eng.timing = (enable & MSPLAT_TIMING_EVENTS) != 0;
    g_eng.count_pairs = (enable & MSPLAT_TIMING_PAIRS) != 0;
    return MSPLAT_OK;
    API_END
}

int msplat_hip_set_wide_keys(int on) {
    API_BEGIN
    ENSURE_INIT();
    g_eng.wide_keys = on != 0;
    return MSPLAT_OK;
    API_END
}

int msplat_hip_set_loss_form(int form) {
    API_BEGIN
    ENSURE_INIT();
    if (form < 0 || form > 2) {
        set_err("loss form %d: expected 0 (by size), 1 (streaming) or 2 (two-pass)", form);
        return MSPLAT_E_ARG;
    }
    mskern::set_loss_form(form);
    return MSPLAT_OK;
    API_END
}

int msplat_hip_set_log_pool_chunks(int chunks) {
    API_BEGIN
    ENSURE_INIT();
    g_eng.log_init = chunks > 0 ? chunks : 0;
    g_eng.log_cap = 0;
    g_eng.log_valid = false;
    return MSPLAT_OK;
    API_END
}

int msplat_hip_set_deep_tile_len(int len) {
    API_BEGIN
    ENSURE_INIT();
    g_eng.deep_len = len > 0 ? len : kDefaultDeepLen;
    g_eng.deep_len_set = len > 0;
    return MSPLAT_OK;
    API_END
}

int msplat_hip_stage_times(const char **names, float *ms, int max) {
    std::lock_guard<std::mutex> lk(g_mu);
    int k = 0;
    for (int i = 0; i < ST_COUNT && k < max; ++i) {
        if (!g_eng.stage_valid[i]) continue;
        if (names) names[k] = kStageNames[i];
        if (ms) ms[k] = g_eng.stage_ms[i];
        ++k;
    }
    return k;
}

int64_t msplat_hip_last_pairs_evaluated(void) { return g_eng.pairs[0]; }

int msplat_hip_last_raster_counts(int64_t out[5]) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!out) return MSPLAT_E_ARG;
    for (int i = 0; i < 5; ++i) out[i] = g_eng.pairs[i];
    return MSPLAT_OK;
}

int msplat_hip_log_pool_stats(int64_t out[5]) {
    API_BEGIN
    if (!out) return MSPLAT_E_ARG;
    ENSURE_INIT();
    Engine &E = g_eng;
    const msr::BlendLog &L = E.log_desc;
    out[0] = E.log_used;
    out[1] = 0;
    out[2] = E.log_redos;
    out[3] = E.n ? log_worst_chunks(E) : 0;
    out[4] = (int64_t)(E.blend_log.cap + E.t_ckpt.cap + E.log_table.cap + E.wave_cnt.cap + E.log_ctr.cap);
    if (E.log_valid && L.counters) {
        std::vector<int> c((size_t)L.nsub + 1);
        HIPC(hipMemcpyAsync(c.data(), L.counters, c.size() * 4, hipMemcpyDeviceToHost, E.stream));
        HIPC(hipStreamSynchronize(E.stream));
        for (int i = 0; i < L.nsub; ++i) out[1] += c[i];
    }
    return MSPLAT_OK;
    API_END
}

int msplat_hip_check_fast_rcp(int efield_lo, int efield_hi, int64_t *mismatches) {
    API_BEGIN
    if (!mismatches || efield_lo < 1 || efield_hi > 254 || efield_lo > efield_hi) return MSPLAT_E_ARG;
    ENSURE_INIT();
    return check_rcp_locked(efield_lo, efield_hi, mismatches);
    API_END
}

}  // extern "C"
