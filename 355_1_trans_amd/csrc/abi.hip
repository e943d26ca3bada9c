// C ABI of libqgemm.so: argument validation, dispatch, layout helpers.
//
// Host C++ only; every entry point launches asynchronously on the caller's
// stream, allocates nothing and returns a hipError_t (contract of the
// reference launcher, SNAP gemm_a8w8_blockscale_bpreshuffle_launch.cc:29-65).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "launch.hpp"
#include "qgemm.h"
#include "band_gemm.hpp"
#include "bsf32_gemm.hpp"
#include "burst_gemm.hpp"
#include "decode_gemm.hpp"
#include "mid_gemm.hpp"
#include "runs_gemm.hpp"
#include "slice_gemm.hpp"
#include "stream_gemm.hpp"

static_assert(sizeof(opus_gemm_scale_kargs) == 96, "reference kargs ABI is 96 bytes");
static_assert(__builtin_offsetof(opus_gemm_scale_kargs, ptr_sfa) == 64, "reference kargs ABI");
static_assert(__builtin_offsetof(opus_gemm_scale_kargs, stride_sfa) == 80, "reference kargs ABI");
static_assert(__builtin_offsetof(opus_gemm_ldsbypass_kargs, ptr_c) == 24, "ldsbypass kargs ABI");
static_assert(__builtin_offsetof(opus_gemm_mxfp4_scale_kargs, grid_blocks) == 96, "mxfp4 kargs: common block first");

namespace qg {

namespace {
thread_local char g_trace[512];
thread_local size_t g_trace_len;
}  // namespace

const char* g_trace_str() { return g_trace; }

void trace_reset() {
    g_trace_len = 0;
    g_trace[0] = 0;
}

void trace_launch(const char* fmt, ...) {
    if (g_trace_len + 2 >= sizeof(g_trace)) return;
    if (g_trace_len) g_trace[g_trace_len++] = '+';
    va_list ap;
    va_start(ap, fmt);
    const int w = std::vsnprintf(g_trace + g_trace_len, sizeof(g_trace) - g_trace_len, fmt, ap);
    va_end(ap);
    if (w > 0) g_trace_len = std::min(sizeof(g_trace) - 1, g_trace_len + (size_t)w);
    g_trace[g_trace_len] = 0;
}

}  // namespace qg

namespace {

using qg::SkinnyArgs;
using qg::SkinnyKind;
using qg::TileArgs;

constexpr int kMaxDevices = 64;
std::atomic<int> g_arch_ok[kMaxDevices];  // 0 unknown, 1 gfx950, 2 other
std::atomic<int> g_cus[kMaxDevices];      // compute units, 0 = not read yet

// Compute units of the current device: every plan sizes its grid and K
// split to one round of workgroups on this device (256 on MI355X).
int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (dev >= 0 && dev < kMaxDevices) {
        const int known = g_cus[dev].load(std::memory_order_relaxed);
        if (known > 0) return known;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    if (dev >= 0 && dev < kMaxDevices) g_cus[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

// Current device must be gfx950 (SNAP launch.cc:55-61).
hipError_t check_arch() {
    int dev = 0;
    hipError_t st = hipGetDevice(&dev);
    if (st != hipSuccess) return st;
    if (dev >= 0 && dev < kMaxDevices) {
        const int known = g_arch_ok[dev].load(std::memory_order_relaxed);
        if (known == 1) return hipSuccess;
        if (known == 2) return hipErrorInvalidDeviceFunction;
    }
    hipDeviceProp_t props{};
    st = hipGetDeviceProperties(&props, dev);
    if (st != hipSuccess) return st;
    const bool ok = std::strncmp(props.gcnArchName, "gfx950", 6) == 0;
    if (dev >= 0 && dev < kMaxDevices) g_arch_ok[dev].store(ok ? 1 : 2, std::memory_order_relaxed);
    return ok ? hipSuccess : hipErrorInvalidDeviceFunction;
}

// rows*cols*batch*bytes fits in int32 (the kernels use signed 32-bit
// offsets within one batch; SNAP launch.cc:10-15).
bool bounded_count(long long rows, long long cols, long long batch, long long bytes) {
    if (rows <= 0 || cols <= 0 || batch <= 0) return false;
    const long long limit = INT_MAX / bytes;
    if (rows > limit / cols) return false;
    return batch <= limit / (rows * cols);
}

bool overlaps(const void* a, uint64_t a_bytes, const void* b, uint64_t b_bytes) {
    const auto ba = reinterpret_cast<uintptr_t>(a);
    const auto bb = reinterpret_cast<uintptr_t>(b);
    return ba < bb + b_bytes && bb < ba + a_bytes;
}

// Bytes spanned by a strided batch of `rows` rows of `pitch` elements.
uint64_t span(long long batch, long long batch_stride, long long rows, long long pitch, long long last_row_len,
              long long elem) {
    if (rows <= 0) return 0;
    return (uint64_t)(((batch - 1) * batch_stride + (rows - 1) * pitch + last_row_len) * elem);
}

// a >= 0, b > 0; no intermediate past a (a + b - 1 overflows near INT_MAX)
int ceil_div(int a, int b) { return a / b + (a % b != 0); }

// Elements per aligned vector store of C: the largest power of two (at
// most 16 bytes) whose byte size divides ptr_c, the row pitch and, for
// batch > 1, the batch stride.
int c_vec_elems(const opus_gemm_scale_kargs& a, int out_elem) {
    uintptr_t bits = reinterpret_cast<uintptr_t>(a.ptr_c) | (uintptr_t)((long long)a.stride_c * out_elem);
    if (a.batch > 1) bits |= (uintptr_t)((long long)a.stride_c_batch * out_elem);
    int align = 16;
    while (align > out_elem && (bits & (uintptr_t)(align - 1))) align >>= 1;
    return align / out_elem;
}

void fill_common(TileArgs& t, const opus_gemm_scale_kargs& a, int kbytes, int out_elem) {
    t.a = static_cast<const uint8_t*>(a.ptr_a);
    t.b = static_cast<const uint8_t*>(a.ptr_b);
    t.c = a.ptr_c;
    t.sfa = static_cast<const uint8_t*>(a.ptr_sfa);
    t.sfb = static_cast<const uint8_t*>(a.ptr_sfb);
    t.m = a.m;
    t.n = a.n;
    t.kbytes = kbytes;
    t.lda = a.stride_a;
    t.ldb = a.stride_b;
    t.ldc = a.stride_c;
    t.c_vec = c_vec_elems(a, out_elem);
    t.a_batch = a.stride_a_batch;
    t.b_batch = a.stride_b_batch;
    t.c_batch = a.stride_c_batch;
    t.sfa_batch = a.stride_sfa_batch;
    t.sfb_batch = a.stride_sfb_batch;
    t.tiles_m = ceil_div(a.m, 256);
    t.tiles_n = ceil_div(a.n, 256);
    t.group_m = 4;
    t.unit_scale = 127;
}

bool flag01(int v) { return v == 0 || v == 1; }

// 16-byte MX scale panels need 16-byte aligned scale rows and whole panels
// (K/32 a multiple of 16, i.e. K % 512 == 0).
bool mx_wide_panels(const opus_gemm_scale_kargs& a) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a.ptr_sfa), pb = reinterpret_cast<uintptr_t>(a.ptr_sfb);
    return a.k % 512 == 0 && (pa & 15) == 0 && (pb & 15) == 0 && a.stride_sfa % 16 == 0 && a.stride_sfb % 16 == 0 &&
           (a.batch == 1 || (a.stride_sfa_batch % 16 == 0 && a.stride_sfb_batch % 16 == 0));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// The kernels move A/B rows with 16-byte DMAs and scales with 4-byte DMAs.
bool dma_aligned(const opus_gemm_scale_kargs& a, bool scales_dword) {
    if (!aligned(a.ptr_a, 16) || !aligned(a.ptr_b, 16) || a.stride_a % 16 || a.stride_a_batch % 16 ||
        a.stride_b_batch % 16)
        return false;
    if (scales_dword && (!aligned(a.ptr_sfa, 4) || !aligned(a.ptr_sfb, 4)))
        return false;
    return true;
}

// ---------------------------------------------------------------- split-K plan
// Skinny-M problems (too few 256 x 256 tiles to fill the GPU) run on the
// skinny kernel (one 8-wave workgroup per CU).  One CU streams ~50 GB/s, so
// HBM bandwidth needs most of the 256 CUs busy: the plan takes the widest N
// tile (64, 32 or 16 columns) that gives at least kMinTiles workgroups.  When
// even 16-column tiles give fewer than kSplitBelow, K is split across
// workgroups -- only up to one round of workgroups (cus), keeping >= 16
// K-tiles per slice and the fp32 partials below a quarter of B's bytes.  This
// plan depends on the shape only, so its workspace query and its launch
// always agree (the MX entries' four-wave K split also depends on the
// workspace bytes passed: see plan_wide_ws).
constexpr int kMinTiles = 192;
constexpr int kSplitBelow = 128;
// Split-K counters sit in a fixed block at the start of the workspace (the
// 2048 bytes the workspace contract names); a fixed size keeps the counters
// of any later call clear of earlier calls' partials.  A split needs one
// counter per output tile, so splits are planned only up to kMaxCounters tiles.
constexpr size_t kCounterBytes = 2048;
constexpr long long kMaxCounters = kCounterBytes / sizeof(unsigned);
static_assert(kSplitBelow <= kMaxCounters, "counter block too small");
// Each split launch tags its counters with a fresh 24-bit epoch
// (qg::split_arrive, common.hpp), so arrivals are counted from zero whatever
// a counter word held before: a workspace needs no clearing, and one left
// mid-count (an interrupted launch) or never zeroed cannot make a slice
// take itself for the last.  Launches that share a workspace are
// stream-ordered, so consecutive epochs never meet on one word.
std::atomic<unsigned> g_epoch{0};
unsigned next_epoch() { return (g_epoch.fetch_add(1u, std::memory_order_relaxed) + 1u) & 0xffffffu; }
// the counter word's arrival count is 8 bits: no plan splits K more ways
constexpr int kMaxSplit = 255;

struct Plan {
    bool skinny = false;
    bool decode = false;     // skinny shape with M <= 64 on an LDS-staged B layout
    bool mid = false;        // fp32 block scales on 128 x 128 tiles (mid_gemm.hpp)
    int mb = 1, nb = 1, nw = 8, m_tiles = 1, n_tiles = 1, splitk = 1, kt_per_split = 1;
    size_t ctr_bytes = 0, ws_bytes = 0;
};

// Decode plan (M <= 64): workgroups of nw waves own 16*nw columns and all
// rows.  K is split while the tiles leave more than half of the CUs idle,
// keeping >= kDecodeMinKt K-tiles per slice and the fp32 partials below a
// quarter of B's bytes; of 8 and 4 waves the one that puts more workgroups
// in flight wins (8 on a tie: A is shared by more columns).
constexpr int kDecodeMinKt = 8;

void plan_decode(Plan& p, int m, int n, int k_tiles, int batch, long long b_bytes, int cus) {
    p.decode = true;
    p.mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    p.m_tiles = 1;
    long long best = -1;
    for (int nw : {8, 4}) {
        const long long tiles = (long long)ceil_div(n, 16 * nw) * batch;
        long long split = 1;
        if (tiles < cus / 2 && tiles <= kMaxCounters &&
            (long long)m * n < (1LL << 29)) {    // partial offsets are 32-bit bytes
            split = std::min<long long>(cus / tiles, k_tiles / kDecodeMinKt);
            split = std::min<long long>(split, b_bytes / (16LL * m * n));
            split = std::max<long long>(std::min<long long>(split, kMaxSplit), 1);
        }
        const int kt_per = ceil_div(k_tiles, (int)split);
        const int sk = ceil_div(k_tiles, kt_per);
        const long long wgs = tiles * sk;
        if (wgs > best) {
            best = wgs;
            p.nw = nw;
            p.n_tiles = ceil_div(n, 16 * nw);
            p.kt_per_split = kt_per;
            p.splitk = sk;
        }
    }
    if (p.splitk > 1) {
        p.ctr_bytes = kCounterBytes;    // split only below cus / 2 tiles
        p.ws_bytes = p.ctr_bytes + (size_t)p.splitk * batch * m * n * 4;
    } else {
        p.kt_per_split = k_tiles;
    }
}

// decode_ok: the B layout can go through the decode kernel's LDS stages.
// The decode kernel (waves split N, A shared through LDS) runs the fp8
// decode shapes whose N is too narrow for the skinny kernel without a K
// split; with enough N tiles the skinny kernel (waves split K) streams
// row-major B with better DRAM page locality and needs no split.
// decode_wide: the B layout streams well through the decode kernel's LDS
// stages (the K-panel B', 16-row K-tiles of 2 KB), which then also takes
// M >= 16 with up to 2 * kSplitBelow skinny tiles and >= 32 K-tiles: A is
// shared by the workgroup's waves instead of re-read by every 16-column
// skinny tile (BS fp32 M = 64: N = 2112, K = 7168 17.8 -> 14.8 us; N = 7168,
// K = 16384 39.7 -> 33.0 us; N = 8192, K = 7168, M = 48 / 64: 19.0 / 21.1 ->
// 17.6 / 19.3 us; M = 1 or short K stay faster on the skinny
// kernel, and row-major B (MXFP8) on the skinny kernel at any M).  Short K
// (<= 16 K-tiles) with many skinny tiles goes to the decode kernel for
// either layout: the skinny kernel's 8 waves would share too few K-tiles
// (N = 24576, K = 1536, BS fp32 M = 1, 16, 64: 11.9, 13.0, 22.6 -> 10.7,
// 11.2, 17.3 us; MXFP8 M = 16, 64: 15.0, 23.9 -> 11.9, 19.6 us; with 224
// tiles, N = 7168, K = 2048, the skinny kernel wins)
// decode_short: the short-K rule alone (MXFP4, which the decode kernel
// otherwise streams slower than the skinny kernel; M = 16, 32 with 12-16
// K-tiles: 16.7, 13.6 -> 14.0, 12.6 us, M = 64 alike)
Plan plan_gemm(int m, int n, int k_tiles, int batch, long long b_bytes, int cus, bool force_skinny,
               bool decode_ok = true, bool decode_wide = false, bool decode_short = false) {
    Plan p;
    const long long tiles256 = (long long)ceil_div(m, 256) * ceil_div(n, 256) * batch;
    p.skinny = force_skinny || (m <= 256 && tiles256 < 128);
    p.kt_per_split = k_tiles;
    if (!p.skinny) return p;
    p.mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    p.m_tiles = ceil_div(m, 16 * p.mb);
    for (int nb = 4; nb >= 1; nb /= 2) {
        p.nb = nb;
        p.n_tiles = ceil_div(n, 16 * nb);
        if ((long long)p.n_tiles * p.m_tiles * batch >= kMinTiles) break;
    }
    const long long base = (long long)p.n_tiles * p.m_tiles * batch;
    const bool short_k = k_tiles <= 16 && base >= 2 * kSplitBelow;
    if (m <= 64 && ((decode_ok && (base < kSplitBelow || short_k ||
                                   (decode_wide && m >= 16 && base <= 2 * kSplitBelow && k_tiles >= 32))) ||
                    (decode_short && short_k))) {
        plan_decode(p, m, n, k_tiles, batch, b_bytes, cus);
        return p;
    }
    if (base >= kSplitBelow) return p;
    if ((long long)m * n >= (1LL << 29)) return p;    // partial offsets are 32-bit bytes
    long long split = cus / base;
    split = std::min<long long>(split, k_tiles / 16);
    split = std::min<long long>(split, b_bytes / (16LL * m * n));
    split = std::min<long long>(split, kMaxSplit);
    if (split <= 1) return p;
    p.kt_per_split = ceil_div(k_tiles, (int)split);
    p.splitk = ceil_div(k_tiles, p.kt_per_split);
    if (p.splitk > 1) {
        p.ctr_bytes = kCounterBytes;    // base < kSplitBelow counters
        p.ws_bytes = p.ctr_bytes + (size_t)p.splitk * batch * m * n * 4;
    }
    return p;
}

// fp32 block scales: M <= kMidMinM keeps the decode / skinny plan; larger M
// runs the 256 x 256 kernel once it has at least kMidBelow tiles, else the
// 128 x 128 kernel, with K split until about 2 * cus workgroups (two per
// CU) are in flight -- cus (one per CU) when the tiles alone split K at
// least in two -- with >= kMidMinKt K-tiles per slice; where K has >= 24
// K-tiles or the tiles are one M tile, slices down to kMidMinKtDeep while
// one round of workgroups (one per CU) holds them.
constexpr int kMidMinM = 64;
constexpr int kMidBelow = 128;
constexpr int kMidMinKt = 16;
constexpr int kMidMinKtDeep = 8;

// M <= 256 with at least kMidBelow 256 x 256 tiles (N > 32512 at batch 1):
// the planners below replace the 256 x 256 plan of small M there, and the
// burst kernel stays out for M > 16 (N = 32768 - 129280, M = 17-32: the
// 128 x 128 kernel 1.05-1.4x faster)
bool wide_region(int n, int batch) { return (long long)ceil_div(n, 256) * batch >= kMidBelow; }

// A 256 x 256 plan the small-M rule replaces: M <= 128, or M <= 192 with
// K <= 2048 and fewer 256 x 256 tiles than CUs (measured, N = 32768 -
// 129280: the 128 x 128 kernel 1.1-1.7x faster for M <= 128; for M = 192
// only while the 256 x 256 tiles leave CUs idle, 0.8-0.9x past that)
bool small_m_wide(int m, int n, int batch, long long k, int cus) {
    const long long tiles256 = (long long)ceil_div(m, 256) * ceil_div(n, 256) * batch;
    return m <= 128 || (m <= 192 && k <= 2048 && tiles256 < cus);
}

// Replaces p with a 128 x 128 plan when M > kMidMinM and the 256 x 256
// kernel would have fewer than kMidBelow tiles (always with force).
void plan_mid(Plan& p, int m, int n, int k_tiles, int batch, int cus, bool force = false) {
    if (m <= kMidMinM && !force) return;
    const long long tiles256 = (long long)ceil_div(m, 256) * ceil_div(n, 256) * batch;
    if (tiles256 >= kMidBelow && !force) return;
    p = Plan{};
    p.mid = true;
    p.kt_per_split = k_tiles;
    const long long tiles = (long long)ceil_div(m, 128) * ceil_div(n, 128) * batch;
    const long long target = 2LL * cus;    // two workgroups per CU
    if (tiles >= target / 2 || (long long)m * n >= (1LL << 29))    // 32-bit partial offsets
        return;
    long long split = std::min<long long>(target / tiles, k_tiles / kMidMinKt);
    // up to cus / 2 tiles: at most one workgroup per CU (four LDS stages,
    // longer slices, fewer partials) -- N = 7168, K = 16384: MXFP8 M = 128
    // 75.0 -> 61.9 us, BS fp32 M = 128 64.9 -> 47.0, M = 256 76.5 -> 64.0,
    // MXFP4 M = 256 54.7 -> 50.7; shapes with less K unchanged
    if (cus / tiles >= 2) split = std::min<long long>(split, cus / tiles);
    // 8-K-tile slices (the slices summed by splitk_reduce_kernel): BS fp32
    // M = 128, N = 2112, K = 7168 22.4 -> 17.7 us, MXFP4 M = 128 - 512,
    // K = 7168 (28 K-tiles, unsplit before) 1.2-1.75x, MXFP8 M = 128,
    // K = 2048 1.15-1.3x; K = 2048 at M >= 256, or a second round of
    // workgroups, up to 1.6x slower
    if (k_tiles >= 24 || ceil_div(m, 128) == 1)
        split = std::max<long long>(split, std::min<long long>(cus / tiles, k_tiles / kMidMinKtDeep));
    if (split <= 1) return;
    p.kt_per_split = ceil_div(k_tiles, (int)split);
    p.splitk = ceil_div(k_tiles, p.kt_per_split);
    if (p.splitk > 1) {
        p.ctr_bytes = kCounterBytes;    // unused by this kernel: keeps the partials past the counter block
        p.ws_bytes = p.ctr_bytes + (size_t)p.splitk * batch * m * n * 4;
    }
}

// Burst kernel (burst_gemm.hpp) for fp32-block-scale decode shapes: its own
// cost-model plan when that plan is accepted; workspace = counters +
// splitk * batch * M * N fp32 partials when K is split.
qg::BurstPlan plan_bsf32_burst(int m, int n, int k_tiles, int batch) {
    if (m > 16 && wide_region(n, batch)) return qg::BurstPlan{};
    return qg::burst_plan(m, n, k_tiles, batch, device_cus(), kMaxCounters);
}

size_t burst_ws_bytes(const qg::BurstPlan& b, int m, int n, int batch) {
    return b.ok && b.splitk > 1 ? kCounterBytes + (size_t)b.splitk * batch * m * n * 4 : 0;
}

hipError_t run_burst(const TileArgs& t, int batch, const qg::BurstPlan& pl, bool frag, long long b_bytes, bool bf16,
                     void* ws, hipStream_t stream) {
    qg::BurstArgs a{};
    a.t = t;
    a.splitk = pl.splitk;
    a.kt_per_split = pl.kt_per_split;
    a.n_tiles = pl.n_tiles;
    a.b_bytes = b_bytes;
    if (pl.splitk > 1) {    // the caller brought the workspace (checked before routing)
        a.counters = static_cast<unsigned*>(ws);
        a.epoch = next_epoch();
        a.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kCounterBytes);
    }
    return qg::launch_burst(a, frag, pl.mb, pl.nb, pl.waves, batch, bf16, stream);
}

Plan plan_bsf32(int m, int n, int k_tiles, int batch, long long b_bytes, bool decode_ok) {
    const int cus = device_cus();
    Plan p = plan_gemm(m, n, k_tiles, batch, b_bytes, cus, false, decode_ok, decode_ok);
    // 64 < M <= 128: half of every 256-row tile would be padding, so the
    // 128 x 128 kernel even with many tiles (M = 128, N = 65536, K = 1536:
    // 30.2 -> 25.7 us); also at exactly kMidBelow 256 x 256 tiles, half a
    // round, with >= 12 K-tiles (M = 4096, N = 2048, K = 7168: 70.3 -> 65.0
    // us; M = 1024, N = 8192, K = 1536: 20.5 -> 18.3 us; M = 256,
    // N = 32768, K = 512 stays on 256 x 256 tiles, 11.7 vs 13.3 us; from
    // 168 tiles the 256 x 256 kernel is 1.3-1.45x faster)
    const long long tiles256 = (long long)ceil_div(m, 256) * ceil_div(n, 256) * batch;
    plan_mid(p, m, n, k_tiles, batch, cus,
             m > kMidMinM && (m <= 128 || (tiles256 == kMidBelow && k_tiles >= 12)));
    if (p.mid && m <= 320) {
        // one round of skinny workgroups (3/4 to all of the CUs, no K split),
        // each streaming <= 512 KB of A and B, beats the 128 x 128 kernel's
        // K split (N = 7168, K = 3072, M = 128: 21.9 -> 17.7 us; N = 8192,
        // K = 1536, M = 128); at 570-690 KB per workgroup (N = 1536 / 2048,
        // K = 7168, M = 66-312) the 128 x 128 kernel with its separately
        // reduced deep split is 1.05-1.4x faster, and more bytes or a
        // second round of skinny workgroups favour it further
        const Plan s = plan_gemm(m, n, k_tiles, batch, b_bytes, cus, true, false);
        const long long wgs = (long long)s.n_tiles * s.m_tiles * batch;
        const long long wg_bytes = 16LL * (s.mb + s.nb) * k_tiles * 128;
        if (s.splitk == 1 && wgs <= cus && 4 * wgs >= 3LL * cus && wg_bytes <= 512 * 1024) p = s;
    }
    // long K (>= 128 K-tiles) where the 128 x 128 plan would run unsplit:
    // the 256 x 256 kernel, whose tail split (plan_tail) fills the CUs
    // (dsv4, N = 7168, K = 16384 / 21504, M = 768 / 1024: 1.13-1.25x)
    if (p.mid && p.splitk == 1 && k_tiles >= 128 && m > 512) p = Plan{};
    // M <= 64 and >= 128 256 x 256 tiles (N > 32512): the 256-row tiles
    // would be mostly padding -- the 128 x 128 kernel (N = 32768 - 129280,
    // M = 33-64: 1.3-1.6x; also M = 192 with K <= 2048 and fewer 256 x 256
    // tiles than CUs: N = 32768, K = 1536 1.08x), or for M <= 32 with
    // K > 2048 the skinny kernel unsplit (N = 32768 - 129280, K = 7168:
    // within 5% of the fastest id, 1.35-1.7x over the 256 x 256 tiles)
    if (!p.skinny && !p.mid && small_m_wide(m, n, batch, (long long)k_tiles * 128, cus)) {
        if (m <= 32 && k_tiles > 16) p = plan_gemm(m, n, k_tiles, batch, b_bytes, cus, true, decode_ok, decode_ok);
        else plan_mid(p, m, n, k_tiles, batch, cus, true);
    }
    // M = 17-64 whose 128 x 128 tiles alone fill 3/4 of the CUs (N >= 24576
    // at batch 1): M = 33-64 the 128 x 128 kernel, which reads B once at full
    // occupancy (N = 24576, K = 1024 - 7168: 1.2-1.4x over the decode and
    // skinny kernels); M = 17-32 on K-panel B the decode kernel, whose waves
    // share A (N = 24576 - 32768, K = 2048 - 7168: 1.05-1.25x over the skinny
    // and 128 x 128 kernels)
    const long long tiles128 = (long long)ceil_div(m, 128) * ceil_div(n, 128) * batch;
    if (m > 16 && m <= kMidMinM && 4 * tiles128 >= 3LL * cus) {
        if (m > 32) {
            if (!p.mid) plan_mid(p, m, n, k_tiles, batch, cus, true);
        } else if (decode_ok && k_tiles > 8) {
            p = Plan{};
            p.skinny = true;
            plan_decode(p, m, n, k_tiles, batch, b_bytes, cus);
        }
    }
    // M = 17-64 whose skinny plan spills a little past one round (1 to 1.5
    // rounds) while the 128 x 128 tiles fill half of the CUs: the 128 x 128
    // kernel (N = 20480, K = 4096-16384: 1.07-1.74x; M = 32, K = 4096 the
    // decode kernel is another 9% faster). Two full rounds stay skinny
    // (ldsbypass M = 32, N = 32768, K = 7168: the fastest id)
    const long long skinny_wgs = (long long)p.n_tiles * p.m_tiles * batch * p.splitk;
    if (p.skinny && !p.decode && m > 16 && m <= kMidMinM && 2 * tiles128 >= cus && skinny_wgs > cus &&
        2 * skinny_wgs < 3LL * cus)
        plan_mid(p, m, n, k_tiles, batch, cus, true);
    return p;
}

// Tail split of the 256 x 256 fp32-scale kernel (bsf32_gemm.hpp): one
// workgroup per CU, so batch x tiles beyond whole rounds of `cus` leave a
// partial last round; its tiles may be cut into S K-slices (one workgroup
// each, fp32 partial images summed by the last slice).  Cost model in
// microseconds, fitted to the dsv4 sweep run both ways (bsf32 kernel, 27
// shapes with a tail): a K-tile takes kTailKtFreeUs on a CU while few CUs
// run and kTailKtFullUs when the chip is at its power limit, so the tail
// costs max(its longest workgroup, its total work at the full-load rate);
// a split adds its partial images, written and read back at
// kTailPartialBytesPerUs (256 KB each way per slice), and kTailFixUs.  The
// split is taken when it saves at least 5%: K >= 16384 with a tail of
// 80-108 tiles gains 5-12% (M = 3072, N = 7168, K = 16384: 347 -> 311 us);
// larger tails lose to the chip's power limit (M = 2048, N = 7168,
// K = 16384 split 8 ways: 195 -> 611 us) and short K to the partial traffic.
// Workspace = counters + the tail's partial images.
struct TailPlan {
    int dp = 0, split = 1, kps = 0;
    size_t ws_bytes = 0;
};
constexpr double kTailKtFreeUs = 1.27, kTailKtFullUs = 1.5, kTailFixUs = 3.4, kTailPartialBytesPerUs = 2.0e6;
constexpr int kTailMaxSplit = 8, kTailMinKt = 4;

TailPlan plan_tail(int m, int n, int k_tiles, int batch, int cus) {
    TailPlan tp;
    const long long items = (long long)ceil_div(m, 256) * ceil_div(n, 256) * batch;
    tp.dp = (int)std::min<long long>(items, 1LL << 30);
    tp.kps = k_tiles;
    const long long tail = items % cus;
    if (tail == 0 || items >= (1LL << 30) || tail > kMaxCounters) return tp;
    const double power = (double)tail * k_tiles / cus * kTailKtFullUs;
    const double unsplit = std::max((double)k_tiles * kTailKtFreeUs, power);
    double best = unsplit;
    int bs = 1;
    for (int sp = 2; sp <= kTailMaxSplit; ++sp) {
        const int kps = ceil_div(k_tiles, sp);
        if (kps < kTailMinKt) break;
        if (ceil_div(k_tiles, kps) != sp) continue;
        const double path = (double)((tail * sp + cus - 1) / cus) * kps * kTailKtFreeUs;
        const double c = std::max(path, power) + (double)tail * sp * 2 * 256 * 256 * 4 / kTailPartialBytesPerUs +
                         kTailFixUs;
        if (c < 0.95 * unsplit && c < best) {
            best = c;
            bs = sp;
        }
    }
    if (bs == 1) return tp;
    tp.dp = (int)(items - tail);
    tp.split = bs;
    tp.kps = ceil_div(k_tiles, bs);
    tp.ws_bytes = kCounterBytes + (size_t)tail * bs * 256 * 256 * sizeof(float);
    return tp;
}

// Kernel routes of the fp32 block-scale entries (QGEMM_KID_* in qgemm.h):
// AUTO resolves to one of the others by the plans above; a forced route
// runs that kernel with its own plan (tile shape and K split), or fails
// with hipErrorInvalidValue where the kernel cannot take the shape.  The
// workspace a route needs is the same with or without one at hand (the
// query); without one, split plans run unsplit.
struct BsfRoute {
    int kid = QGEMM_KID_AUTO;
    bool ok = false;
    qg::BurstPlan bp;
    Plan pl;
    TailPlan tp;
    size_t ws_bytes = 0;
};

BsfRoute route_bsf32(int m, int n, int k_tiles, int batch, long long b_bytes, bool frag, int kid, bool have_ws) {
    BsfRoute r;
    r.kid = kid;
    if (m <= 0 || n <= 0 || k_tiles <= 0 || batch <= 0) return r;
    const int cus = device_cus();
    switch (kid) {
        case QGEMM_KID_AUTO: {
            r.bp = plan_bsf32_burst(m, n, k_tiles, batch);
            if (r.bp.ok) {
                r.ws_bytes = burst_ws_bytes(r.bp, m, n, batch);
                if (r.bp.splitk == 1 || have_ws) {
                    r.kid = QGEMM_KID_BURST;
                    r.ok = true;
                    return r;
                }
            }
            r.pl = plan_bsf32(m, n, k_tiles, batch, b_bytes, !frag);
            r.kid = r.pl.mid ? QGEMM_KID_MID
                             : r.pl.skinny ? (r.pl.decode ? QGEMM_KID_DECODE : QGEMM_KID_SKINNY) : QGEMM_KID_TILE256;
            if (r.kid == QGEMM_KID_TILE256) r.tp = plan_tail(m, n, k_tiles, batch, cus);
            if (!r.bp.ok) r.ws_bytes = r.kid == QGEMM_KID_TILE256 ? r.tp.ws_bytes : r.pl.ws_bytes;
            r.ok = true;
            return r;
        }
        case QGEMM_KID_TILE256:
            r.tp = plan_tail(m, n, k_tiles, batch, cus);
            r.ws_bytes = r.tp.ws_bytes;
            r.ok = true;
            return r;
        case QGEMM_KID_MID:
            plan_mid(r.pl, m, n, k_tiles, batch, cus, true);
            break;
        case QGEMM_KID_SKINNY:
            r.pl = plan_gemm(m, n, k_tiles, batch, b_bytes, cus, true, false);
            break;
        case QGEMM_KID_DECODE:
            if (m > 64 || frag) return r;    // the decode kernel stages K-panel B' only
            r.pl.skinny = true;
            plan_decode(r.pl, m, n, k_tiles, batch, b_bytes, cus);
            break;
        case QGEMM_KID_BURST:
            r.bp = qg::burst_plan(m, n, k_tiles, batch, cus, kMaxCounters, false);
            if (!r.bp.ok) return r;
            r.ws_bytes = burst_ws_bytes(r.bp, m, n, batch);
            if (r.bp.splitk > 1 && !have_ws) r.bp = qg::burst_plan(m, n, k_tiles, batch, cus, kMaxCounters, false, 1);
            r.ok = r.bp.ok;
            return r;
        default:
            return r;
    }
    r.ws_bytes = r.pl.ws_bytes;
    r.ok = true;
    return r;
}

// MX: the same 128 x 128 rule (row-major B, E8M0 scales applied by the
// MFMA); small M on >= 128 256 x 256 tiles runs the 128 x 128 kernel
// (N = 32768 - 129280, MXFP4 / MXFP8 M = 24-128: 1.1-1.7x over the
// 256 x 256 tiles), M <= 16 the skinny kernel unsplit (MXFP8 K = 7168,
// M = 16: 85.3 -> 49.4 us at N = 32768)
Plan plan_mx(int m, int n, int k_tiles, int batch, long long b_bytes, bool fp4) {
    const int cus = device_cus();
    auto skinny = [&](bool force) {
        return fp4 ? plan_gemm(m, n, k_tiles, batch, b_bytes, cus, force, false, false, true)
                   : plan_gemm(m, n, k_tiles, batch, b_bytes, cus, force);
    };
    Plan p = skinny(false);
    // M > 256: the 128 x 128 kernel below 96 256 x 256 tiles, and up to
    // kMidBelow (inclusive) only with short K (<= 16 K-tiles fp8, <= 12
    // fp4); longer K from 96 tiles runs the 256 x 256 kernel (M = 512-1024,
    // N = 6144-12288, K = 2048-7168: 128 x 128 1.03-1.2x slower there,
    // 1.1-1.3x faster with short K; N = 8192, M = 1024, K = 1536 MXFP4
    // 18.6 -> 14.0 us)
    const long long tiles256 = (long long)ceil_div(m, 256) * ceil_div(n, 256) * batch;
    const bool short_k = k_tiles <= (fp4 ? 12 : 16);
    if (m <= 256 || tiles256 < 96 || (tiles256 <= kMidBelow && short_k))
        plan_mid(p, m, n, k_tiles, batch, cus, m > 256 && tiles256 == kMidBelow);
    if (!p.skinny && !p.mid && small_m_wide(m, n, batch, (long long)k_tiles * (fp4 ? 256 : 128), cus)) {
        if (m <= 16) p = skinny(true);
        else plan_mid(p, m, n, k_tiles, batch, cus, true);
    }
    // M = 33-64 whose 128 x 128 tiles alone fill 3/8 of the CUs: the
    // 128 x 128 kernel reads B once at full occupancy where the decode and
    // skinny kernels re-stream it per row group (N = 24576, M = 64, K =
    // 1024-4096, MXFP4 / MXFP8: 1.3-1.6x over them; N = 12288 - 16384,
    // M = 48 / 64, K = 7168 / 16384: MXFP8 1.05-1.17x, MXFP4 1.02-1.14x).
    // M = 17-32 where the skinny plan spills into a second round and the
    // 128 x 128 tiles fill half of the CUs (N = 20480, K = 7168 / 16384:
    // 1.4-1.6x; one round at N = 16384 stays skinny)
    const long long tiles128 = (long long)ceil_div(m, 128) * ceil_div(n, 128) * batch;
    const long long skinny_wgs = (long long)p.n_tiles * p.m_tiles * batch * p.splitk;
    if (p.skinny && m > 32 && m <= kMidMinM && 8 * tiles128 >= 3LL * cus) plan_mid(p, m, n, k_tiles, batch, cus, true);
    else if (p.skinny && m > 16 && m <= 32 && skinny_wgs > cus && 2 * tiles128 >= cus)
        plan_mid(p, m, n, k_tiles, batch, cus, true);
    return p;
}

// Row-streaming decode kernel (stream_gemm.hpp): M <= kStreamMaxM with
// row-major MX B.  One MFMA covers wr rows of B and wr rows of A (a quarter
// of its products are used at wr = 4, a sixteenth at wr = 1), so wr grows
// with M; past M = 8 the 16-row fragments of the skinny kernel waste less
// matrix work.  A's K slice sits in LDS; when all of K does not fit, K is
// split over workgroups (fp32 partials in the workspace, like the skinny
// kernel's split).  The plan depends on the shape only, so the workspace
// query and the launch agree.
constexpr int kStreamMaxM = 8;
constexpr int kStreamMinN = 256;

struct StreamPlan {
    bool ok = false;
    int wr = 1, mb = 1, splitk = 1, seg_per_split = 1, rows = 1;
    size_t ws_bytes = 0;
};

StreamPlan plan_stream(int m, int n, int k, int batch, bool fp4) {
    StreamPlan p;
    if (m > kStreamMaxM || n < kStreamMinN) return p;
    // measured at N = 7168, K = 16384 (MXFP4 / MXFP8 us): M = 4 wr 1, 2, 4:
    // 15.8, 14.5, 14.0 / 23.6, 22.0, 22.2; M = 8 wr 2, 4: 18.0, 15.6 / 24.4,
    // 22.5 (skinny kernel: 16.7 / 24.9); M = 2 wr 1 and 2 alike
    if (m == 1) { p.wr = 1; p.mb = 1; }
    else if (m == 2) { p.wr = 2; p.mb = 2; }
    else { p.wr = 4; p.mb = m <= 4 ? 4 : 8; }
    const int seg = (fp4 ? 1024 : 2048) / p.wr;
    const int nseg = ceil_div(fp4 ? k / 2 : k, seg);
    const int cap = qg::stream_seg_cap(fp4, p.wr, p.mb);
    p.splitk = ceil_div(nseg, cap);
    p.seg_per_split = ceil_div(nseg, p.splitk);
    p.splitk = ceil_div(nseg, p.seg_per_split);
    // about one workgroup per CU; rows bounded by the waves' row groups and
    // by the LDS image of their B scales
    const long long nblk_target = std::max<long long>(1, device_cus() / ((long long)p.splitk * batch));
    long long rows = (n + nblk_target - 1) / nblk_target;
    const int wsp = 1 << qg::stream_ws_log2(p.seg_per_split * 64 / p.wr);
    const long long rcap = std::min(qg::stream_max_rows(p.wr), qg::kStreamWsBytes / wsp);
    if (rows > rcap) {
        // more than one round: the rows spread evenly over whole rounds (at
        // the cap, N = 16384 would be 293 blocks -- a second round of 37)
        const long long rounds = ((n + rcap - 1) / rcap + nblk_target - 1) / nblk_target;
        rows = (n + rounds * nblk_target - 1) / (rounds * nblk_target);
    }
    p.rows = (int)std::max<long long>(rows, 1);
    if (p.splitk > kMaxSplit) return p;
    if (p.splitk > 1) {
        const long long blocks = (long long)ceil_div(n, p.rows) * batch;
        if (blocks > (long long)(kCounterBytes / sizeof(unsigned)) || (long long)m * n >= (1LL << 29)) return p;
        p.ws_bytes = kCounterBytes + (size_t)p.splitk * batch * m * n * 4;
    }
    p.ok = true;
    return p;
}

bool stream_ok(const opus_gemm_scale_kargs& a, bool fp4) {
    if (!plan_stream(a.m, a.n, a.k, a.batch, fp4).ok) return false;
    if (!dma_aligned(a, false) || a.stride_b % 16 || !aligned(a.ptr_sfa, 4) || a.stride_sfa % 4) return false;
    return a.batch == 1 || a.stride_sfa_batch % 4 == 0;
}

// Band kernel (band_gemm.hpp): M <= 64 with row-major MX B.  A workgroup
// owns 128 * cb columns and a K slice of at most band_kt_max(mb) K-tiles
// (its A in LDS); the plan takes the (cb, split) whose workgroups fill the
// most CUs in one round, the smaller split on a tie, and no plan when even
// the smallest split needs more than one round.
struct BandPlan {
    bool ok = false;
    int mb = 1, cb = 1, splitk = 1, kps = 1, bands = 1;
    size_t ws_bytes = 0;
};

BandPlan plan_band(int m, int n, int k_tiles, int batch) {
    BandPlan best;
    if (m < 1 || m > 64 || n < 1 || k_tiles < 1 || batch < 1) return best;
    const int cus = device_cus();
    const int mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    const int ktm = qg::band_kt_max(mb);
    long long best_wgs = 0;
    for (int cb : {1, 2}) {
        if (mb == 2 && cb == 2) continue;    // no LDS room for a ring
        const int bands = ceil_div(n, qg::band_cols(cb));
        for (int sk = ceil_div(k_tiles, ktm); sk <= k_tiles; ++sk) {
            const int kps = ceil_div(k_tiles, sk);
            const int sp = ceil_div(k_tiles, kps);
            if (sp != sk) continue;
            const long long wgs = (long long)bands * sp * batch;
            if (wgs > cus || sp > kMaxSplit) break;
            if (sp > 1 && ((long long)bands * batch > kMaxCounters || (long long)m * n >= (1LL << 29))) break;
            if (wgs > best_wgs) {
                best_wgs = wgs;
                best.ok = true;
                best.mb = mb;
                best.cb = cb;
                best.splitk = sp;
                best.kps = kps;
                best.bands = bands;
                best.ws_bytes = sp > 1 ? kCounterBytes + (size_t)sp * batch * m * n * 4 : 0;
            }
        }
    }
    return best;
}

// operands the band kernel's DMAs take: 16-byte rows of A and B, dword
// scale rows of both operands
bool band_ok(const opus_gemm_scale_kargs& a) {
    if (!dma_aligned(a, true) || a.stride_b % 16 || a.stride_sfa % 4 || a.stride_sfb % 4) return false;
    return a.batch == 1 || (a.stride_sfa_batch % 4 == 0 && a.stride_sfb_batch % 4 == 0);
}

hipError_t run_band(const BandPlan& bp, const TileArgs& t, int batch, bool fp4, bool bf16, void* ws,
                    hipStream_t stream) {
    qg::BandArgs b{};
    b.t = t;
    b.splitk = bp.splitk;
    b.kt_per_split = bp.kps;
    b.bands = bp.bands;
    if (bp.splitk > 1) {    // the caller brought the workspace (checked before routing)
        b.counters = static_cast<unsigned*>(ws);
        b.epoch = next_epoch();
        b.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kCounterBytes);
    }
    return qg::launch_band(b, fp4, bp.mb, bp.cb, batch, bf16, stream);
}

// Launches the stream kernel; false when its K split needs a workspace the
// call did not bring (the caller then runs the skinny kernel).
bool run_stream(const TileArgs& t, int k, int batch, bool fp4, bool bf16, void* ws, size_t ws_bytes,
                hipStream_t stream, hipError_t* st) {
    const StreamPlan pl = plan_stream(t.m, t.n, k, batch, fp4);
    qg::StreamArgs s{};
    s.t = t;
    s.rows_per_wg = pl.rows;
    s.splitk = pl.splitk;
    s.seg_per_split = pl.seg_per_split;
    if (pl.splitk > 1) {
        if (!ws || ws_bytes < pl.ws_bytes || !aligned(ws, 256)) return false;
        s.counters = static_cast<unsigned*>(ws);
        s.epoch = next_epoch();
        s.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kCounterBytes);
    }
    *st = qg::launch_stream(s, fp4, pl.wr, pl.mb, batch, bf16, stream);
    return true;
}

// Wide-kernel MX scale panels: with a workspace, both operands' E8M0
// scales are first copied into the panel-major layout [K/32/pb][rows][pb],
// so that each panel DMA reads 1 KB contiguously (row-major rows put every
// lane of a panel DMA on its own cache line: MXFP8 8192^3 ran 4.4% slower).
// Without one, the wide kernel reads the row-major scales directly.
size_t round256(size_t b) { return (b + 255) / 256 * 256; }
size_t scale_panel_bytes(const opus_gemm_scale_kargs& a) {
    if (a.k % 512) return 0;
    const size_t kg = (size_t)a.k / 32;
    return kCounterBytes + round256((size_t)a.batch * a.m * kg) + round256((size_t)a.batch * a.n * kg);
}

// Launches the wide MX kernel (panel width pb, kt_bytes scale bytes per
// K-tile and row), through the panel-major copy when the workspace holds it.
// Copies both operands' row-major E8M0 scales into the panel-major layout
// [K/32/pb][rows][pb] after the workspace's counter block and points t at
// it (per-K-tile stride rows * kt_bytes, batch strides whole planes).
hipError_t copy_scale_panels(TileArgs& t, const opus_gemm_scale_kargs& a, int pb, int kt_bytes, void* ws,
                             hipStream_t stream) {
    const int kg = a.k / 32;
    uint8_t* pa = static_cast<uint8_t*>(ws) + kCounterBytes;
    uint8_t* pbp = pa + round256((size_t)a.batch * a.m * kg);
    qg::ScalePanelArgs sp{};
    sp.src[0] = t.sfa;
    sp.src[1] = t.sfb;
    sp.dst[0] = pa;
    sp.dst[1] = pbp;
    sp.rows[0] = a.m;
    sp.rows[1] = a.n;
    sp.ld[0] = a.stride_sfa;
    sp.ld[1] = a.stride_sfb;
    sp.src_batch[0] = a.stride_sfa_batch;
    sp.src_batch[1] = a.stride_sfb_batch;
    sp.dst_batch[0] = (long long)a.m * kg;
    sp.dst_batch[1] = (long long)a.n * kg;
    sp.ngroups = kg;
    sp.pb = pb;
    const hipError_t st = qg::launch_mx_scale_panels(sp, a.batch, stream);
    if (st != hipSuccess) return st;
    t.sfa = pa;
    t.sfb = pbp;
    t.sfa_sm = pb;
    t.sfb_sn = pb;
    t.sfa_sk = a.m * kt_bytes;
    t.sfb_sk = a.n * kt_bytes;
    t.sfa_batch = sp.dst_batch[0];
    t.sfb_batch = sp.dst_batch[1];
    return hipSuccess;
}

// The one-by-four wave MXFP4 kernel reads its scales in e8m0_shuffle order
// (per 32-row block and K-tile 256 contiguous bytes): the row-major entry
// shuffles both operands' scales into the workspace, [A: batch x
// ceil(M/32) x 32 x K/32][B: batch x ceil(N/32) x 32 x K/32] (each part
// 256-byte aligned), and the kernel reads them from there.
size_t quad_plane_bytes(int rows, int k) { return (size_t)ceil_div(rows, 32) * 32 * (size_t)(k / 32); }
size_t quad_scale_bytes(const opus_gemm_scale_kargs& a) {
    return round256((size_t)a.batch * quad_plane_bytes(a.m, a.k)) + round256((size_t)a.batch * quad_plane_bytes(a.n, a.k));
}
// Both operands' scales into the workspace's shuffled planes: one launch.
qg::ShuffleArgs quad_shuffle_args(const opus_gemm_scale_kargs& a, const uint8_t* sfa, const uint8_t* sfb, void* ws) {
    qg::ShuffleArgs sh{};
    const int kg = a.k / 32, chunks = ceil_div(ceil_div(kg, 8), 16);
    sh.src[0] = sfa;
    sh.src[1] = sfb;
    sh.dst[0] = static_cast<uint8_t*>(ws);
    sh.dst[1] = sh.dst[0] + round256((size_t)a.batch * quad_plane_bytes(a.m, a.k));
    sh.rows[0] = a.m;
    sh.rows[1] = a.n;
    sh.ld[0] = a.stride_sfa;
    sh.ld[1] = a.stride_sfb;
    sh.src_batch[0] = a.stride_sfa_batch;
    sh.src_batch[1] = a.stride_sfb_batch;
    sh.dst_batch[0] = (long long)quad_plane_bytes(a.m, a.k);
    sh.dst_batch[1] = (long long)quad_plane_bytes(a.n, a.k);
    sh.kg = kg;
    sh.units[0] = ceil_div(a.m, 32) * chunks;
    sh.units[1] = ceil_div(a.n, 32) * chunks;
    return sh;
}
hipError_t run_quad(TileArgs t, const opus_gemm_scale_kargs& a, bool bf16, void* ws, hipStream_t stream) {
    const qg::ShuffleArgs sh = quad_shuffle_args(a, t.sfa, t.sfb, ws);
    const hipError_t st = qg::launch_e8m0_shuffle_blocks(sh, a.batch, stream);
    if (st != hipSuccess) return st;
    t.sfa = sh.dst[0];
    t.sfb = sh.dst[1];
    t.sfa_sm = t.sfb_sn = a.k;    // 32 rows x K/32 groups per 32-row block
    t.sfa_batch = sh.dst_batch[0];
    t.sfb_batch = sh.dst_batch[1];
    return qg::launch_quad_mx4(t, a.batch, false, bf16, stream);
}

hipError_t run_wide_mx(TileArgs t, const opus_gemm_scale_kargs& a, bool fp4, int pb, bool bf16, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
    const int kt_bytes = fp4 ? 8 : 4;
    t.sfa_sk = kt_bytes;
    t.sfb_sk = kt_bytes;
    const size_t need = scale_panel_bytes(a);
    if (pb >= 16 && need && ws && ws_bytes >= need && aligned(ws, 256)) {
        const hipError_t st = copy_scale_panels(t, a, pb, kt_bytes, ws, stream);
        if (st != hipSuccess) return st;
    }
    return fp4 ? qg::launch_wide_mx4_raw(t, a.batch, bf16, pb, stream)
               : qg::launch_wide_mx8_raw(t, a.batch, bf16, pb, stream);
}

// The four-wave MX kernel split into s equal K slices (plan_wide_split):
// slice z of the launch's batch reads A / B row bytes [z * slice, (z + 1) *
// slice) and the scales of those groups -- whole panels of the panel-major
// copy when the panels divide the slices (pb >= 16; the copy follows the
// counter block and the planes follow the copy), else the row-major scales
// (the planes follow the counter block) -- and writes fp32 plane z;
// splitk_reduce_kernel then sums the planes in slice order into C.
int wide_split_pb(const opus_gemm_scale_kargs& a, bool fp4, int s);

hipError_t run_wide_split(TileArgs t, const opus_gemm_scale_kargs& a, bool fp4, int s, bool bf16, void* ws,
                          hipStream_t stream) {
    const int slice = a.k / s;                          // K elements per slice
    const int slice_bytes = fp4 ? slice / 2 : slice;    // multiple of 128 (>= kWideSplitMinKt K-tiles)
    const int kt_bytes = fp4 ? 8 : 4;
    const int pb = wide_split_pb(a, fp4, s);
    TileArgs w = t;
    w.kbytes = slice_bytes;
    w.a_batch = slice_bytes;
    w.b_batch = slice_bytes;
    size_t head = kCounterBytes;
    if (pb >= 16) {
        // panel-major copy [K/32/pb][rows][pb]: a slice of whole panels
        // starts (slice / 32) * rows bytes further
        const hipError_t st = copy_scale_panels(w, a, pb, kt_bytes, ws, stream);
        if (st != hipSuccess) return st;
        w.sfa_batch = (long long)(slice / 32) * a.m;
        w.sfb_batch = (long long)(slice / 32) * a.n;
        head = scale_panel_bytes(a);
    } else {
        w.sfa_sk = w.sfb_sk = kt_bytes;    // row-major scales: one K-tile's bytes
        w.sfa_batch = w.sfb_batch = slice / 32;
    }
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + head);
    w.c = part;
    w.ldc = a.n;
    w.c_batch = (long long)a.m * a.n;
    w.c_vec = a.n % 4 == 0 ? 4 : a.n % 2 == 0 ? 2 : 1;
    const hipError_t st = fp4 ? qg::launch_wide_mx4_raw(w, s, false, pb, stream)
                              : qg::launch_wide_mx8_raw(w, s, false, pb, stream);
    if (st != hipSuccess) return st;
    qg::SplitReduceArgs r{};
    r.ws = part;
    r.c = t.c;
    r.m = a.m;
    r.n = a.n;
    r.ldc = t.ldc;
    r.c_vec = t.c_vec;
    r.splitk = s;
    r.batch = 1;
    r.c_batch = t.c_batch;
    return qg::launch_splitk_reduce(r, bf16, stream);
}

// Launches the 128 x 128 kernel; a NULL workspace runs it without a K split.
hipError_t run_mid(TileArgs t, int batch, Plan pl, bool bf16, qg::MidKind kind, void* ws, size_t ws_bytes,
                   int k_tiles, hipStream_t stream) {
    qg::MidArgs a{};
    t.tiles_m = ceil_div(t.m, 128);
    t.tiles_n = ceil_div(t.n, 128);
    a.t = t;
    if (pl.splitk > 1 && ws) {
        if (ws_bytes < pl.ws_bytes || !aligned(ws, 256)) return hipErrorInvalidValue;
        a.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + pl.ctr_bytes);
        a.splitk = pl.splitk;
        a.kt_per_split = pl.kt_per_split;
    } else {
        a.splitk = 1;
        a.kt_per_split = k_tiles;
    }
    // at most one workgroup per CU (the K split's minimum slice bounds it):
    // four LDS stages, three K-tiles in flight; else two workgroups per CU
    // with two stages each
    const long long wgs = (long long)t.tiles_m * t.tiles_n * batch * a.splitk;
    return qg::launch_mid(a, batch, bf16, kind, wgs <= device_cus() ? 4 : 2, stream);
}

// Launches the skinny or decode kernel.  A NULL workspace runs one K slice
// (no partials); a non-NULL one must hold plan.ws_bytes and be 256-byte
// aligned.
hipError_t run_skinny(SkinnyKind kind, const TileArgs& t, int batch, Plan pl, bool bf16, void* ws,
                      size_t ws_bytes, int k_tiles, hipStream_t stream) {
    unsigned* counters = nullptr;
    float* partials = nullptr;
    if (pl.splitk > 1 && ws) {
        if (ws_bytes < pl.ws_bytes || !aligned(ws, 256)) return hipErrorInvalidValue;
        counters = static_cast<unsigned*>(ws);
        partials = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + pl.ctr_bytes);
    } else {
        pl.splitk = 1;
        pl.kt_per_split = k_tiles;
    }
    if (pl.decode) {
        qg::DecodeArgs d{};
        d.t = t;
        d.ws = partials;
        d.counters = counters;
        d.epoch = next_epoch();
        d.splitk = pl.splitk;
        d.kt_per_split = pl.kt_per_split;
        d.n_tiles = pl.n_tiles;
        return qg::launch_decode(kind, d, pl.mb, pl.nw, batch, bf16, stream);
    }
    SkinnyArgs s{};
    s.t = t;
    s.counters = counters;
    s.epoch = next_epoch();
    s.ws = partials;
    s.splitk = pl.splitk;
    s.kt_per_split = pl.kt_per_split;
    s.n_tiles = pl.n_tiles;
    s.m_tiles = pl.m_tiles;
    // per-wave scale panels when a wave's run fits one 64-byte panel row and
    // the 16-byte DMAs stay aligned (skinny_gemm.hpp); fp32 scales need
    // row-major row scales (K-tiles contiguous)
    {
        const bool mx = kind == SkinnyKind::MX8_RAW || kind == SkinnyKind::MX4_RAW;
        const int kt_bytes = kind == SkinnyKind::MX4_RAW ? 8 : 4;
        const int unit = mx ? 1 : 4;    // bytes per stride / batch-stride count
        const bool layout = mx || t.sfa_sk == 1;
        const bool aligned16 = aligned(t.sfa, 16) && aligned(t.sfb, 16) && (t.sfa_sm * unit) % 16 == 0 &&
                               (t.sfb_sn * unit) % 16 == 0 &&
                               (batch == 1 || ((t.sfa_batch * unit) % 16 == 0 && (t.sfb_batch * unit) % 16 == 0));
        const int run = qg::skinny_panel_run(pl.kt_per_split, qg::kSkinnyWaves, kt_bytes);
        s.scale_panel = layout && aligned16 && qg::skinny_scp_fits(pl.mb, pl.nb, mx) && run * kt_bytes <= 64 &&
                        ceil_div(pl.kt_per_split, run) >= 6 &&    // keep most waves busy
                        (pl.splitk == 1 || pl.kt_per_split % (16 / kt_bytes) == 0);
    }
    return qg::launch_skinny(kind, s, pl.mb, pl.nb, batch, bf16, stream);
}

hipError_t run_bsf32(const BsfRoute& r, const TileArgs& t, int batch, bool frag, long long b_bytes, bool bf16,
                     void* ws, size_t ws_bytes, int k_tiles, hipStream_t stream) {
    switch (r.kid) {
        case QGEMM_KID_BURST:
            return run_burst(t, batch, r.bp, frag, b_bytes, bf16, ws, stream);
        case QGEMM_KID_MID:
            return run_mid(t, batch, r.pl, bf16, frag ? qg::MidKind::BS_FRAG : qg::MidKind::BS_KPANEL, ws, ws_bytes,
                           k_tiles, stream);
        case QGEMM_KID_SKINNY:
        case QGEMM_KID_DECODE:
            return run_skinny(frag ? SkinnyKind::BSF32_FRAG : SkinnyKind::BSF32_KPANEL, t, batch, r.pl, bf16, ws,
                              ws_bytes, k_tiles, stream);
        default: {
            // the eight-wave kernel with VGPR accumulators and a VALU rescale
            // per K-tile (bsf32_gemm.hpp); the tail split only with the
            // workspace at hand
            qg::Bsf32Args a{};
            a.t = t;
            a.dp_tiles = t.tiles_m * t.tiles_n * batch;
            a.tail_split = 1;
            a.kt_per_split = k_tiles;
            if (r.tp.split > 1 && ws && ws_bytes >= r.tp.ws_bytes) {
                a.dp_tiles = r.tp.dp;
                a.tail_split = r.tp.split;
                a.kt_per_split = r.tp.kps;
                a.counters = static_cast<unsigned*>(ws);
                a.epoch = next_epoch();
                a.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kCounterBytes);
            }
            return qg::launch_bsf32(a, batch, bf16, frag, stream);
        }
    }
}

// Kernel routes of the MX entries (QGEMM_KID_*): AUTO follows the plans
// above (row-streaming kernel for M <= 8, burst kernel where its gate
// accepts, skinny / decode, 128 x 128, 256 x 256 tiles); a forced id runs
// that family with its own plan or fails for shapes it cannot take.
// Row-run kernel (runs_gemm.hpp): M <= 64, row-major MX B read in 512-byte
// runs of each row.  32 columns per workgroup; K slices of at most 64
// K-tiles (16 stages), more slices while a round of workgroups leaves more
// than a quarter of the CUs idle and each slice keeps >= 16 K-tiles; a split
// needs the workspace (counters + fp32 partial planes).
struct RunsPlan {
    bool ok = false;
    int mb = 1, splitk = 1, kt_per_split = 1, n_tiles = 1;
    size_t ws_bytes = 0;
};
RunsPlan plan_runs(int m, int n, int kt, int batch, int cus, bool have_ws) {
    RunsPlan r;
    if (m < 1 || m > 64 || n < 1 || kt < 1 || batch < 1) return r;
    r.mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    r.n_tiles = ceil_div(n, qg::kRunsCols);
    const long long tiles = (long long)r.n_tiles * batch;
    constexpr int kMaxSlice = 16 * qg::kRunsStage;
    int split = ceil_div(kt, kMaxSlice);
    if (have_ws)
        while (tiles * split * 4 < 3LL * cus && ceil_div(kt, split + 1) >= 16) ++split;
    const int kps = ceil_div(ceil_div(kt, split), qg::kRunsStage) * qg::kRunsStage;
    split = ceil_div(kt, kps);
    if (split > 1) {
        if (!have_ws || tiles > kMaxCounters || (long long)m * n >= (1LL << 29)) return r;
        r.ws_bytes = kCounterBytes + (size_t)split * batch * m * n * 4;
    }
    r.splitk = split;
    r.kt_per_split = kps;
    r.ok = true;
    return r;
}
// Slice kernel (slice_gemm.hpp): M <= 64; 16 slice_nbw(mb) columns per
// workgroup and K slices of slice_kps(mb) K-tiles (A's slice is 128 KB of
// LDS); a split needs the workspace.
RunsPlan plan_slice(int m, int n, int kt, int batch, bool have_ws) {
    RunsPlan r;
    if (m < 1 || m > 64 || n < 1 || kt < 1 || batch < 1) return r;
    r.mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    r.n_tiles = ceil_div(n, 16 * qg::slice_nbw(r.mb));
    const long long tiles = (long long)r.n_tiles * batch;
    const int kps = qg::slice_kps(r.mb);
    const int split = ceil_div(kt, kps);
    if (split > 255) return r;    // the counters' 8-bit arrival count
    if (split > 1) {
        if (!have_ws || tiles > kMaxCounters || (long long)m * n >= (1LL << 29)) return r;
        r.ws_bytes = kCounterBytes + (size_t)split * batch * m * n * 4;
    }
    r.splitk = split;
    r.kt_per_split = kps;
    r.ok = true;
    return r;
}
// its loads take 16 bytes of A / B rows and of scale rows per lane
bool runs_ok(const opus_gemm_scale_kargs& a) {
    if (!dma_aligned(a, false) || a.stride_b % 16 || !aligned(a.ptr_sfa, 16) || !aligned(a.ptr_sfb, 16) ||
        a.stride_sfa % 16 || a.stride_sfb % 16)
        return false;
    return a.batch == 1 || (a.stride_sfa_batch % 16 == 0 && a.stride_sfb_batch % 16 == 0);
}

struct MxRoute {
    int kid = QGEMM_KID_AUTO;
    bool ok = false;
    Plan pl;
    StreamPlan sp;
    qg::BurstPlan bp;
    BandPlan bd;
    RunsPlan rn;
    int wsplit = 1;    // K slices of the four-wave kernel (plan_wide_split)
    size_t ws_bytes = 0;
};

// K split of the four-wave MX kernel (batch 1) where its 256 x 256 tiles
// leave at least half of the CUs idle: the K slices run as batch entries of
// the unchanged kernel (A / B / scale batch strides of one slice's bytes
// along K, row-major scales, fp32 output into partial planes) and
// splitk_reduce_kernel sums them.  Slices of >= kWideSplitMinKt K-tiles,
// equal (the slice count divides the K-tiles).  The slices read the
// scale-panel copy when the panels divide them (whole panels per slice),
// else row-major scales.  M = 512-1024, N = 6144-12288 at 96-128 tiles:
// MXFP8 K = 7168 (28-K-tile slices) 1.07-1.2x, K = 16384 1.35-1.49x;
// MXFP4 K = 16384 1.16-1.18x; 16-K-tile slices (K = 4096) ran 4-17%
// slower than the unsplit kernel, and MXFP4 on row-major scales 0.87-1.05x
// against its unsplit kernel on 32-byte panels, so it splits only on
// panels.
constexpr int kWideSplitMinKt = 24;
// panel width of a split into s slices: 16 (fp8) / 32 or 16 (fp4) when the
// panels divide the slices, else the row-major widths 4 / 8
int wide_split_pb(const opus_gemm_scale_kargs& a, bool fp4, int s) {
    const int kt_bytes = fp4 ? 8 : 4;
    const int pb = fp4 ? (a.k % 1024 == 0 ? 32 : 16) : 16;
    const int slice_kt = a.k / (fp4 ? 256 : 128) / s;
    return mx_wide_panels(a) && slice_kt % (pb / kt_bytes) == 0 ? pb : kt_bytes;
}
int plan_wide_split(const opus_gemm_scale_kargs& a, bool fp4, int cus) {
    if (a.batch != 1 || (long long)a.m * a.n >= (1LL << 29)) return 1;
    const int kt = a.k / (fp4 ? 256 : 128);
    const long long tiles = (long long)ceil_div(a.m, 256) * ceil_div(a.n, 256);
    int s = (int)std::min<long long>(cus / tiles, kt / kWideSplitMinKt);
    while (s > 1 && kt % s) --s;
    if (s > 1 && fp4 && wide_split_pb(a, fp4, s) < 16) return 1;
    return std::max(s, 1);
}
// [counters | scale panels (when used) | s fp32 partial planes]
size_t wide_split_bytes(const opus_gemm_scale_kargs& a, bool fp4, int s) {
    if (s <= 1) return 0;
    const size_t head = wide_split_pb(a, fp4, s) >= 16 ? scale_panel_bytes(a) : kCounterBytes;
    return head + (size_t)s * a.m * a.n * 4;
}
// The four-wave kernel's workspace: the split's partial planes when they fit
// the caller's workspace (ws_cap), else the scale-panel copy.
void plan_wide_ws(MxRoute& r, const opus_gemm_scale_kargs& a, bool fp4, int cus, size_t ws_cap) {
    const int s = plan_wide_split(a, fp4, cus);
    const size_t sb = wide_split_bytes(a, fp4, s);
    r.wsplit = s > 1 && sb <= ws_cap ? s : 1;
    r.ws_bytes = std::max(scale_panel_bytes(a), r.wsplit > 1 ? sb : 0);
}

// Burst plan for MX row-major B: the fp32-block-scale gate, and only up to
// 32 K-tiles (4 KB of K per row) and past M = kStreamMaxM.  Measured
// (graph-replayed, MXFP4 / MXFP8 us): short K gains 1.1-1.5x over the skinny
// kernel (fp4 M = 32: N = 24576, K = 1536 12.4 -> 9.4; N = 7168, K = 2048
// 8.1 -> 5.6; fp8 M = 16, N = 24576, K = 1536 15.6 -> 10.7), long K loses
// (fp4 configs[4] K = 16384, M = 16 / 32: 15.8 / 19.2 on the skinny kernel,
// 17.7 / 29.2 as a burst); M <= 8 stays on the row-streaming kernel, whose
// contiguous row runs 16-row fragments cannot match (M = 1: 12.8 vs 17.5),
// up to N = kStreamBurstN: past it the burst kernel's many short workgroups
// win (N = 16384 - 129280, K = 1536 / 7168: 1.0-1.5x, one shape 4% slower)
constexpr int kStreamBurstN = 16384;

qg::BurstPlan plan_mx_burst(int m, int n, int k_tiles, int batch, bool gate) {
    if (gate && ((m <= kStreamMaxM && n < kStreamBurstN) || k_tiles > 32 || (m > 16 && wide_region(n, batch))))
        return qg::BurstPlan{};
    return qg::burst_plan(m, n, k_tiles, batch, device_cus(), kMaxCounters, gate, 16, true);
}

MxRoute route_mx(const opus_gemm_scale_kargs& a, bool fp4, int kid, bool have_ws, size_t ws_cap) {
    MxRoute r;
    r.kid = kid;
    if (a.m <= 0 || a.n <= 0 || a.k <= 0 || a.batch <= 0 || a.k % (fp4 ? 256 : 128)) return r;
    const int kt = a.k / (fp4 ? 256 : 128);
    const long long bb = (long long)a.n * (fp4 ? a.k / 2 : a.k);
    const int cus = device_cus();
    switch (kid) {
        case QGEMM_KID_AUTO: {
            r.pl = plan_mx(a.m, a.n, kt, a.batch, bb, fp4);
            r.sp = plan_stream(a.m, a.n, a.k, a.batch, fp4);
            r.bp = plan_mx_burst(a.m, a.n, kt, a.batch, true);
            if (r.pl.mid && a.m > 128 && have_ws) {
                // M > 128 on a 128 x 128 plan: the four-wave kernel's K
                // split where its slices fill >= 9/16 of the CUs (M = 512 /
                // 768, N = 6144 / 8192, K = 12288 / 16384: 1.4-1.6x over the
                // 128 x 128 kernel MXFP8, 1.15-1.35x MXFP4 at 144 workgroups;
                // M = 160-256, N = 24576: MXFP8 1.35-1.42x, MXFP4 K = 16384
                // 1.16-1.26x; 96-128 workgroups within 8% either way)
                const int s = plan_wide_split(a, fp4, cus);
                const long long tiles = (long long)ceil_div(a.m, 256) * ceil_div(a.n, 256);
                if (s > 1 && 16 * tiles * s >= 9LL * cus && wide_split_bytes(a, fp4, s) <= ws_cap) r.pl = Plan{};
            }
            if (!r.pl.skinny && !r.pl.mid) plan_wide_ws(r, a, fp4, cus, have_ws ? ws_cap : 0);
            r.ws_bytes = std::max({r.sp.ok ? r.sp.ws_bytes : 0, r.pl.ws_bytes, burst_ws_bytes(r.bp, a.m, a.n, a.batch),
                                   r.pl.skinny || r.pl.mid ? 0 : r.ws_bytes});
            r.ok = true;
            if (a.m > 16 && a.m <= 32 && have_ws && band_ok(a)) {
                // 32-row band plans with long K slices (>= 12 K-tiles) over
                // 7/10 or more of the CUs, where the slice kernel would split
                // K: 128 columns of B per workgroup read once, with A's slice
                // in LDS (graph-replayed, two boxes: MXFP4 configs[4] M = 32
                // 16.7-18.2 us against 18.9-19.8 for the slice kernel and
                // 18.6-20.5 for the skinny one; M = 24 / 32, N = 4096-8192,
                // K = 8192 / 16384, both formats: 8-20% faster than the
                // slice kernel; unsplit slice plans, N = 12288-16384, keep
                // the slice kernel, 1.16x over these band plans)
                const BandPlan bd = plan_band(a.m, a.n, kt, a.batch);
                const RunsPlan sl = runs_ok(a) ? plan_slice(a.m, a.n, kt, a.batch, true) : RunsPlan{};
                const long long wgs = (long long)bd.bands * bd.splitk * a.batch;
                if (bd.ok && bd.splitk > 1 && bd.kps >= 12 && 10 * wgs >= 7LL * cus && (!sl.ok || sl.splitk > 1)) {
                    r.bd = bd;
                    r.kid = QGEMM_KID_BAND;
                    r.ws_bytes = std::max(r.ws_bytes, bd.ws_bytes);
                    return r;
                }
            }
            if (a.m > 8 && runs_ok(a)) {
                // the slice kernel where its plan is one round of 7/10 to all
                // of the CUs with full K slices (or one slice >= 85% full):
                // its B streams straight into registers and A's slice is read
                // once per workgroup (graph-replayed, 96 shapes M = 9-64 x N =
                // 2112-24576 x K = 4096-16384, both formats: 1.03-1.47x on the
                // shapes this takes, e.g. MXFP4 M = 64, N = 7168, K = 16384
                // 26.6 -> 24.6 us, M = 16 16.8 -> 14.2, M = 64, N = 24576,
                // K = 4096 22.4 -> 15.2, MXFP8 M = 32, N = 4096, K = 16384
                // 24.2 -> 20.0; a second sweep of the 109 shapes of a DeepSeek-
                // like grid this rule took: geometric mean 1.13x, up to 1.5x,
                // one MXFP8 shape 5% slower (M = 24, N = 8192, K = 8192); at two
                // rounds or short slices it lost up to 1.8x, and 64-row plans
                // split in two at N = 12288-16384 lost 3-11% to the band
                // kernel, so those keep the plans below)
                const RunsPlan sl = plan_slice(a.m, a.n, kt, a.batch, have_ws);
                if (sl.ok) {
                    const int kps = qg::slice_kps(sl.mb);
                    const long long wgs = (long long)sl.n_tiles * sl.splitk * a.batch;
                    const bool full = kt % kps == 0 || (sl.splitk == 1 && 20 * kt >= 17 * kps);
                    if (10 * wgs >= 7LL * cus && wgs <= cus && full && !(sl.mb == 4 && sl.splitk == 2)) {
                        r.rn = sl;
                        r.kid = QGEMM_KID_SLICE;
                        r.ws_bytes = std::max(r.ws_bytes, sl.ws_bytes);
                        return r;
                    }
                }
            }
            if (a.m > 40 && a.m <= 64 && kt >= 64 && (long long)ceil_div(a.n, qg::kRunsCols) * a.batch <= 128 &&
                have_ws && runs_ok(a)) {
                // the row-run kernel at narrow N and long K, M = 41-64: its
                // 32-column tiles split K to fill the CUs while reading B in
                // 512-byte row runs (graph-replayed, M = 48 / 56 / 64, N =
                // 2112 / 4096, K = 16384: MXFP4 1.04-1.26x, MXFP8 1.14-1.38x
                // over the skinny plans, e.g. MXFP8 M = 64, N = 2112 36.8 ->
                // 26.6 us; at N = 7168 it is within 4% either way, at N =
                // 16384 or K <= 7168 up to 1.5x slower: not taken there)
                const RunsPlan rn = plan_runs(a.m, a.n, kt, a.batch, cus, true);
                if (rn.ok) {
                    r.rn = rn;
                    r.kid = QGEMM_KID_RUNS;
                    r.ws_bytes = std::max(r.ws_bytes, rn.ws_bytes);
                    return r;
                }
            }
            if (a.m > 16 && band_ok(a)) {
                // the band kernel when one unsplit round of bands covers
                // three quarters of the CUs: it reads each B row once with
                // A's slice in LDS and no partials (MXFP4 / MXFP8, N =
                // 24576-32768, K <= 4096, M = 24-64: 1.05-2.1x over the
                // burst / decode / 128 x 128 plans); its split plans lose
                // to them where N is narrow (up to 1.75x slower at N =
                // 8192) and win while N's 128-column strips cover 3/8 to
                // 3/4 of the CUs (N = 12288 - 20480, K = 4096 / 7168,
                // M = 32-64: up to 1.34x, a few shapes within 8% of the
                // best id; wider N keeps the 128 x 128 kernel, the best id
                // measured at N = 24576 / 32768)
                const BandPlan bd = plan_band(a.m, a.n, kt, a.batch);
                const long long bands = (long long)bd.bands * a.batch;
                const long long strips = (long long)ceil_div(a.n, 128) * a.batch;
                if (bd.ok && ((bd.splitk == 1 && 4 * bands >= 3LL * cus) || (bd.splitk > 1 && 8 * strips >= 3LL * cus && 4 * strips < 3LL * cus)) &&
                    (bd.splitk == 1 || have_ws)) {
                    r.bd = bd;
                    r.kid = QGEMM_KID_BAND;
                    r.ws_bytes = std::max(r.ws_bytes, bd.ws_bytes);
                    return r;
                }
            }
            if (r.bp.ok && (r.bp.splitk == 1 || have_ws)) {
                r.kid = QGEMM_KID_BURST;
                return r;
            }
            if (stream_ok(a, fp4)) {
                // without the K split's workspace: the skinny kernel (plan_mx
                // plans it for every M <= 16)
                r.kid = r.sp.splitk == 1 || have_ws ? QGEMM_KID_STREAM : QGEMM_KID_SKINNY;
                return r;
            }
            r.kid = r.pl.mid ? QGEMM_KID_MID
                             : r.pl.skinny ? (r.pl.decode ? QGEMM_KID_DECODE : QGEMM_KID_SKINNY) : QGEMM_KID_TILE256;
            return r;
        }
        case QGEMM_KID_TILE256:
            plan_wide_ws(r, a, fp4, cus, have_ws ? ws_cap : 0);
            break;
        case QGEMM_KID_MID:
            plan_mid(r.pl, a.m, a.n, kt, a.batch, cus, true);
            r.ws_bytes = r.pl.ws_bytes;
            break;
        case QGEMM_KID_SKINNY:
            r.pl = plan_gemm(a.m, a.n, kt, a.batch, bb, cus, true, false);
            r.ws_bytes = r.pl.ws_bytes;
            break;
        case QGEMM_KID_DECODE:
            if (a.m > 64) return r;
            r.pl.skinny = true;
            plan_decode(r.pl, a.m, a.n, kt, a.batch, bb, cus);
            r.ws_bytes = r.pl.ws_bytes;
            break;
        case QGEMM_KID_BURST:
            r.bp = plan_mx_burst(a.m, a.n, kt, a.batch, false);
            if (!r.bp.ok) return r;
            r.ws_bytes = burst_ws_bytes(r.bp, a.m, a.n, a.batch);
            if (r.bp.splitk > 1 && !have_ws)
                r.bp = qg::burst_plan(a.m, a.n, kt, a.batch, cus, kMaxCounters, false, 1, true);
            if (!r.bp.ok) return r;
            break;
        case QGEMM_KID_STREAM:
            if (!stream_ok(a, fp4)) return r;
            r.sp = plan_stream(a.m, a.n, a.k, a.batch, fp4);
            r.ws_bytes = r.sp.ws_bytes;
            if (r.sp.splitk > 1 && !have_ws) return r;    // the row-streaming kernel needs its split
            break;
        case QGEMM_KID_BAND:
            if (!band_ok(a)) return r;
            r.bd = plan_band(a.m, a.n, kt, a.batch);
            if (!r.bd.ok) return r;
            r.ws_bytes = r.bd.ws_bytes;
            if (r.bd.splitk > 1 && !have_ws) return r;    // its K slices need the workspace
            break;
        case QGEMM_KID_QUAD:
            if (!fp4) return r;
            r.ws_bytes = quad_scale_bytes(a);
            if (!have_ws) return r;    // the shuffled scales live in the workspace
            break;
        case QGEMM_KID_RUNS:
            if (!runs_ok(a)) return r;
            r.rn = plan_runs(a.m, a.n, kt, a.batch, cus, have_ws);
            if (!r.rn.ok) return r;
            r.ws_bytes = r.rn.ws_bytes;
            break;
        case QGEMM_KID_SLICE:
            if (!runs_ok(a)) return r;
            r.rn = plan_slice(a.m, a.n, kt, a.batch, have_ws);
            if (!r.rn.ok) return r;
            r.ws_bytes = r.rn.ws_bytes;
            break;
        default:
            return r;
    }
    r.ok = true;
    return r;
}

hipError_t run_mx(const MxRoute& r, TileArgs t, const opus_gemm_scale_kargs& a, bool fp4, bool bf16, void* ws,
                  size_t ws_bytes, hipStream_t stream) {
    const int kt = a.k / (fp4 ? 256 : 128);
    const SkinnyKind sk = fp4 ? SkinnyKind::MX4_RAW : SkinnyKind::MX8_RAW;
    switch (r.kid) {
        case QGEMM_KID_STREAM: {
            hipError_t st = hipSuccess;
            if (!run_stream(t, a.k, a.batch, fp4, bf16, ws, ws_bytes, stream, &st)) return hipErrorInvalidValue;
            return st;
        }
        case QGEMM_KID_BURST: {
            qg::BurstArgs b{};
            b.t = t;
            b.splitk = r.bp.splitk;
            b.kt_per_split = r.bp.kt_per_split;
            b.n_tiles = r.bp.n_tiles;
            b.b_bytes = (long long)(a.n - 1) * a.stride_b + (fp4 ? a.k / 2 : a.k);
            if (r.bp.splitk > 1) {
                b.counters = static_cast<unsigned*>(ws);
                b.epoch = next_epoch();
                b.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kCounterBytes);
            }
            return qg::launch_burst_mx(b, fp4, r.bp.mb, r.bp.nb, r.bp.waves, a.batch, bf16, stream);
        }
        case QGEMM_KID_RUNS:
        case QGEMM_KID_SLICE: {
            qg::RunsArgs x{};
            x.t = t;
            x.splitk = r.rn.splitk;
            x.kt_per_split = r.rn.kt_per_split;
            x.n_tiles = r.rn.n_tiles;
            x.b_bytes = (long long)(a.n - 1) * a.stride_b + (fp4 ? a.k / 2 : a.k);
            if (r.rn.splitk > 1) {
                x.counters = static_cast<unsigned*>(ws);
                x.epoch = next_epoch();
                x.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kCounterBytes);
            }
            return r.kid == QGEMM_KID_SLICE ? qg::launch_slice(x, fp4, r.rn.mb, a.batch, bf16, stream)
                                            : qg::launch_runs(x, fp4, r.rn.mb, a.batch, bf16, stream);
        }
        case QGEMM_KID_SKINNY:
        case QGEMM_KID_DECODE:
            return run_skinny(sk, t, a.batch, r.pl, bf16, ws, ws_bytes, kt, stream);
        case QGEMM_KID_BAND:
            return run_band(r.bd, t, a.batch, fp4, bf16, ws, stream);
        case QGEMM_KID_QUAD:
            return run_quad(t, a, bf16, ws, stream);
        case QGEMM_KID_MID:
            t.sfa_sk = t.sfb_sk = fp4 ? 8 : 4;
            return run_mid(t, a.batch, r.pl, bf16, fp4 ? qg::MidKind::MX4 : qg::MidKind::MX8, ws, ws_bytes, kt,
                           stream);
        default: {
            if (r.wsplit > 1 && ws) return run_wide_split(t, a, fp4, r.wsplit, bf16, ws, stream);
            // fp8: 16-byte panels (32-byte ones cover 8 K-tiles and measured 1%
            // slower); fp4: 32-byte panels (4 K-tiles, two DMA lanes per scale
            // row) need whole panels, K % 1024 == 0
            const int pb = fp4 ? (mx_wide_panels(a) ? (a.k % 1024 == 0 ? 32 : 16) : 8) : (mx_wide_panels(a) ? 16 : 4);
            return run_wide_mx(t, a, fp4, pb, bf16, ws, ws_bytes, stream);
        }
    }
}

// Byte ranges of a call's operands (C first), for the overlap checks of the
// output and of the workspace.
struct Spans {
    const void* p[6];
    uint64_t bytes[6];
    int n = 0;
    void add(const void* q, uint64_t b) {
        p[n] = q;
        bytes[n++] = b;
    }
    bool overlap_any(const void* q, uint64_t b, int from) const {
        for (int i = from; i < n; ++i)
            if (overlaps(q, b, p[i], bytes[i])) return true;
        return false;
    }
};

// One workspace rule for every entry point and every route: NULL runs
// without a workspace (no K split; wide MX kernels read row-major scales
// directly); a non-NULL workspace must hold the bytes the entry's
// *_workspace_bytes query returns, be 256-byte aligned and overlap neither C
// nor an input.  Checked once, before routing.
hipError_t check_workspace(const void* ws, size_t ws_bytes, size_t need, const Spans& sp) {
    if (!ws || need == 0) return hipSuccess;
    if (ws_bytes < need || !aligned(ws, 256) || sp.overlap_any(ws, need, 0)) return hipErrorInvalidValue;
    return hipSuccess;
}

// Validation shared by the MX entry points: dense or padded row-major A/B,
// row-major scales, C [M, N] with stride_c >= N.
hipError_t validate_mx(const opus_gemm_scale_kargs* args, int out_dtype, int kbytes_per_row, int k_align,
                       Spans* sp) {
    if (!args || !args->ptr_a || !args->ptr_b || !args->ptr_c || !args->ptr_sfa || !args->ptr_sfb ||
        !flag01(out_dtype))
        return hipErrorInvalidValue;
    const auto& a = *args;
    const int kg = a.k / 32;
    if (a.m <= 0 || a.n <= 0 || a.k <= 0 || a.batch <= 0 || a.k % k_align) return hipErrorInvalidValue;
    if (a.stride_a < kbytes_per_row || a.stride_b < kbytes_per_row || a.stride_c < a.n || a.stride_sfa < kg ||
        a.stride_sfb < kg)
        return hipErrorInvalidValue;
    if (!dma_aligned(a, true) || a.stride_b % 16 || a.stride_sfa % 4 || a.stride_sfb % 4 ||
        a.stride_sfa_batch % 4 || a.stride_sfb_batch % 4)
        return hipErrorInvalidValue;
    const long long outb = out_dtype ? 2 : 4;
    if (!aligned(a.ptr_c, (uintptr_t)outb)) return hipErrorInvalidValue;
    if (a.batch > 1 &&
        ((long long)a.stride_a_batch < (long long)a.m * a.stride_a ||
         (long long)a.stride_b_batch < (long long)a.n * a.stride_b ||
         (long long)a.stride_c_batch < (long long)a.m * a.stride_c ||
         (long long)a.stride_sfa_batch < (long long)a.m * a.stride_sfa ||
         (long long)a.stride_sfb_batch < (long long)a.n * a.stride_sfb))
        return hipErrorInvalidValue;
    if (!bounded_count(a.m, a.stride_a, 1, 1) || !bounded_count(a.n, a.stride_b, 1, 1) ||
        !bounded_count(a.m, a.stride_c, 1, outb) || !bounded_count(a.m, a.stride_sfa, 1, 1) ||
        !bounded_count(a.n, a.stride_sfb, 1, 1))
        return hipErrorInvalidValue;
    sp->add(a.ptr_c, span(a.batch, a.stride_c_batch, a.m, a.stride_c, a.n, outb));
    sp->add(a.ptr_a, span(a.batch, a.stride_a_batch, a.m, a.stride_a, kbytes_per_row, 1));
    sp->add(a.ptr_b, span(a.batch, a.stride_b_batch, a.n, a.stride_b, kbytes_per_row, 1));
    sp->add(a.ptr_sfa, span(a.batch, a.stride_sfa_batch, a.m, a.stride_sfa, kg, 1));
    sp->add(a.ptr_sfb, span(a.batch, a.stride_sfb_batch, a.n, a.stride_sfb, kg, 1));
    if (sp->overlap_any(sp->p[0], sp->bytes[0], 1)) return hipErrorInvalidValue;
    return hipSuccess;
}

// fp32 block-scale operands (both B layouts): A [M,K] (stride_a >= K),
// SFA column-major [K/128][M] (stride_sfa >= M) or row-major [M][K/128]
// (stride_sfa == 1), SFB [ceil(N/128)][K/128] (stride_sfb >= K/128), C [M,N].
// B is checked by the caller (b_data, b_bytes_per_batch).  Returns the SFA
// element strides along M and K.
hipError_t validate_bsf32(const opus_gemm_scale_kargs& a, const void* b_data, long long b_bytes_per_batch,
                          int out_dtype, int* sfa_sm, int* sfa_sk, Spans* sp) {
    if (!a.ptr_a || !b_data || !a.ptr_c || !a.ptr_sfa || !a.ptr_sfb || !flag01(out_dtype))
        return hipErrorInvalidValue;
    if (a.m <= 0 || a.n <= 0 || a.k <= 0 || a.batch <= 0 || a.k % 128) return hipErrorInvalidValue;
    const int kg = a.k / 128, nbk = ceil_div(a.n, 128);
    const bool sfa_rowmajor = (a.stride_sfa == 1 && a.m > 1);
    if (a.stride_a < a.k || a.stride_c < a.n || a.stride_sfb < kg || (!sfa_rowmajor && a.stride_sfa < a.m))
        return hipErrorInvalidValue;
    if (!aligned(a.ptr_a, 16) || !aligned(b_data, 16) || a.stride_a % 16 || a.stride_a_batch % 16 ||
        !aligned(a.ptr_sfa, 4) || !aligned(a.ptr_sfb, 4))
        return hipErrorInvalidValue;
    const long long outb = out_dtype ? 2 : 4;
    if (!aligned(a.ptr_c, (uintptr_t)outb)) return hipErrorInvalidValue;
    const long long sfa_span = sfa_rowmajor ? (long long)a.m * kg : (long long)(kg - 1) * a.stride_sfa + a.m;
    if (a.batch > 1 &&
        ((long long)a.stride_a_batch < (long long)a.m * a.stride_a ||
         (long long)a.stride_c_batch < (long long)a.m * a.stride_c || (long long)a.stride_sfa_batch < sfa_span ||
         (long long)a.stride_sfb_batch < (long long)nbk * a.stride_sfb))
        return hipErrorInvalidValue;
    if (!bounded_count(a.m, a.stride_a, 1, 1) || !bounded_count(b_bytes_per_batch, 1, 1, 1) ||
        !bounded_count(a.m, a.stride_c, 1, outb) || !bounded_count(sfa_span, 1, 1, 4) ||
        !bounded_count(nbk, a.stride_sfb, 1, 4))
        return hipErrorInvalidValue;
    sp->add(a.ptr_c, span(a.batch, a.stride_c_batch, a.m, a.stride_c, a.n, outb));
    sp->add(a.ptr_a, span(a.batch, a.stride_a_batch, a.m, a.stride_a, a.k, 1));
    sp->add(a.ptr_sfa, span(a.batch, a.stride_sfa_batch, 1, 0, sfa_span, 4));
    sp->add(a.ptr_sfb, span(a.batch, a.stride_sfb_batch, nbk, a.stride_sfb, kg, 4));
    if (sp->overlap_any(sp->p[0], sp->bytes[0], 1)) return hipErrorInvalidValue;
    *sfa_sm = sfa_rowmajor ? kg : 1;
    *sfa_sk = sfa_rowmajor ? 1 : a.stride_sfa;
    return hipSuccess;
}

// B'' bytes of one batch: 16-row blocks, N padded up to a multiple of 16.
size_t frag_bytes(int n, int k) { return (size_t)ceil_div(n, 16) * 16 * (size_t)k; }

// The 96-byte view of the LDS-bypass arguments with B = B''.
opus_gemm_scale_kargs from_ldsbypass(const opus_gemm_ldsbypass_kargs& l) {
    opus_gemm_scale_kargs a{};
    a.ptr_a = l.ptr_a;
    a.ptr_b = l.ptr_b_pp;
    a.ptr_c = l.ptr_c;
    a.m = l.m;
    a.n = l.n;
    a.k = l.k;
    a.batch = l.batch;
    a.stride_a = l.stride_a;
    a.stride_b = l.stride_b;
    a.stride_c = l.stride_c;
    a.stride_a_batch = l.stride_a_batch;
    a.stride_b_batch = l.stride_b_pp_batch;
    a.stride_c_batch = l.stride_c_batch;
    a.ptr_sfa = l.ptr_sfa;
    a.ptr_sfb = l.ptr_sfb;
    a.stride_sfa = l.stride_sfa;
    a.stride_sfb = l.stride_sfb;
    a.stride_sfa_batch = l.stride_sfa_batch;
    a.stride_sfb_batch = l.stride_sfb_batch;
    return a;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- MXFP8 / MXFP4
static hipError_t mx_entry(const opus_gemm_scale_kargs* args, bool fp4, int out_dtype, int kernel_id,
                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
    qg::trace_reset();
    Spans sp;
    hipError_t st = validate_mx(args, out_dtype, args ? (fp4 ? args->k / 2 : args->k) : 0, fp4 ? 256 : 128, &sp);
    if (st != hipSuccess) return st;
    const auto& a = *args;
    const MxRoute r = route_mx(a, fp4, kernel_id, workspace != nullptr, workspace_bytes);
    if (!r.ok) return hipErrorInvalidValue;
    st = check_workspace(workspace, workspace_bytes, r.ws_bytes, sp);
    if (st != hipSuccess) return st;
    st = check_arch();
    if (st != hipSuccess) return st;
    TileArgs t{};
    fill_common(t, a, fp4 ? a.k / 2 : a.k, out_dtype ? 2 : 4);
    t.sfa_sm = a.stride_sfa;
    t.sfb_sn = a.stride_sfb;
    return run_mx(r, t, a, fp4, out_dtype == QGEMM_OUT_BF16, workspace, workspace_bytes, stream);
}

// ws_cap: the most workspace the caller can bring (the four-wave kernel's
// K split is planned only when its partial planes fit)
static size_t mx_workspace(const opus_gemm_scale_kargs* args, bool fp4, int kernel_id, size_t ws_cap = SIZE_MAX) {
    if (!args) return 0;
    const MxRoute r = route_mx(*args, fp4, kernel_id, true, ws_cap);
    return r.ok ? r.ws_bytes : 0;
}

hipError_t gemm_a8w8_mxfp8(const opus_gemm_scale_kargs* args, int out_dtype, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
    return mx_entry(args, false, out_dtype, QGEMM_KID_AUTO, workspace, workspace_bytes, stream);
}
size_t gemm_a8w8_mxfp8_workspace_bytes(const opus_gemm_scale_kargs* args) {
    return mx_workspace(args, false, QGEMM_KID_AUTO);
}
hipError_t gemm_a8w8_mxfp8_kid(const opus_gemm_scale_kargs* args, int out_dtype, int kernel_id, void* workspace,
                               size_t workspace_bytes, hipStream_t stream) {
    return mx_entry(args, false, out_dtype, kernel_id, workspace, workspace_bytes, stream);
}
size_t gemm_a8w8_mxfp8_kid_workspace_bytes(const opus_gemm_scale_kargs* args, int kernel_id) {
    return mx_workspace(args, false, kernel_id);
}

hipError_t gemm_a4w4_mxfp4(const opus_gemm_scale_kargs* args, int out_dtype, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
    return mx_entry(args, true, out_dtype, QGEMM_KID_AUTO, workspace, workspace_bytes, stream);
}
size_t gemm_a4w4_mxfp4_workspace_bytes(const opus_gemm_scale_kargs* args) {
    return mx_workspace(args, true, QGEMM_KID_AUTO);
}
hipError_t gemm_a4w4_mxfp4_kid(const opus_gemm_scale_kargs* args, int out_dtype, int kernel_id, void* workspace,
                               size_t workspace_bytes, hipStream_t stream) {
    return mx_entry(args, true, out_dtype, kernel_id, workspace, workspace_bytes, stream);
}
size_t gemm_a4w4_mxfp4_kid_workspace_bytes(const opus_gemm_scale_kargs* args, int kernel_id) {
    return mx_workspace(args, true, kernel_id);
}

// ------------------------------------------------ MXFP4, aiter bpreshuffle operands
}  // extern "C"

namespace {

// Route of the aiter-format MXFP4 entry.  AUTO: M <= 64 runs the burst
// kernel (B in shuffle_weight(16,16) order is the 16x16x128 MFMA's operand
// order, streamed as whole 1 KB loads; a K split needs the workspace, so
// without one only unsplit plans) -- its gated plan, else, for M = 33-64,
// the ungated one: the 256-row tiles of the one-by-four wave kernel leave
// most CUs idle at these M (graph-replayed, N = 7168, K = 16384: M = 1-32
// 13-22 us against 68; M = 64 32.8 against 69; N = 2112, K = 7168, M = 64:
// 12.4 against 33.6).  The one-by-four wave kernel takes the rest, and the
// decode shapes whose 256-column tiles fill half the CUs over at most 4
// K-tiles (M = 64, N = 32768, K = 512: 9.7 us against 11.5); a persistent
// grid (grid_blocks > 0) the two-by-two wave kernel.  A forced id runs that
// kernel or fails.
struct Mx4sRoute {
    int kid = QGEMM_KID_AUTO;
    bool ok = false;
    qg::BurstPlan bp;
    RunsPlan sl;       // SLICE
    int qsplit = 1;    // QUAD: K slices (batch 1), fp32 partial planes + splitk_reduce
    size_t ws_bytes = 0;
};
// K split of the one-by-four wave kernel where its 256 x 256 tiles leave
// more than half of the CUs idle (middle M, batch 1): equal slices of at
// least 4 K-tiles, as many as the CUs take while the partial planes (4 bytes
// per output and slice) stay within twice B's bytes (s <= K / 4M), run as
// batch entries of the unchanged kernel into fp32 partial planes that
// splitk_reduce_kernel sums in slice order.  Graph-replayed, us, split /
// unsplit: N = 7168, K = 16384, M = 128 / 256 / 512: 32.6 / 44.1 / 54.0
// against 71.3 / 73.3 / 72.7; N = 2112, K = 7168, M = 128 / 256: 19.7 / 27.0
// against 35.4 / 39.6; M = 1024, N = 4096, K = 7168 split 4 ways (planes 4.6x
// B's bytes) 59.2 against 36.2, hence the bound.
int plan_quad_split(const opus_gemm_mxfp4_scale_kargs& x, int cus) {
    if (x.batch != 1 || (long long)x.m * x.n >= (1LL << 29)) return 1;
    const int kt = x.k / 256;
    const long long tiles = (long long)ceil_div(x.m, 256) * ceil_div(x.n, 256);
    if (2 * tiles >= cus) return 1;
    int s = (int)std::min<long long>({cus / tiles, kt / 4, x.k / (4LL * x.m)});
    while (s > 1 && kt % s) --s;
    return std::max(s, 1);
}
Mx4sRoute route_mx4s(const opus_gemm_mxfp4_scale_kargs& x, int kid, bool have_ws) {
    Mx4sRoute r;
    const int kt = x.k / 256;
    const int cus = device_cus();
    auto burst = [&](bool gate) {
        r.bp = qg::burst_plan(x.m, x.n, kt, x.batch, cus, kMaxCounters, gate, 16, true);
        if (r.bp.ok && r.bp.splitk > 1 && !have_ws) r.bp = qg::burst_plan(x.m, x.n, kt, x.batch, cus, kMaxCounters, gate, 1, true);
        r.ws_bytes = burst_ws_bytes(r.bp, x.m, x.n, x.batch);
        return r.bp.ok;
    };
    switch (kid) {
        case QGEMM_KID_AUTO: {
            r.ok = true;
            const bool quad_short = 2LL * ceil_div(x.n, 256) * x.batch >= cus && kt <= 4;
            if (x.grid_blocks == 0 && x.m > 8 && x.m <= 64) {
                // the slice kernel on the row-major route's rule (one round of
                // 7/10 to all of the CUs, full K slices); W16 makes each of its
                // B fragment loads one 1 KB run
                const RunsPlan sl = plan_slice(x.m, x.n, kt, x.batch, have_ws);
                if (sl.ok) {
                    const int kps = qg::slice_kps(sl.mb);
                    const long long wgs = (long long)sl.n_tiles * sl.splitk * x.batch;
                    const bool full = kt % kps == 0 || (sl.splitk == 1 && 20 * kt >= 17 * kps);
                    if (10 * wgs >= 7LL * cus && wgs <= cus && full) {
                        r.sl = sl;
                        r.kid = QGEMM_KID_SLICE;
                        r.ws_bytes = sl.ws_bytes;
                        return r;
                    }
                }
            }
            if (x.grid_blocks > 0) r.kid = QGEMM_KID_TILE256;
            else if (x.m <= 64 && !quad_short && (burst(true) || (x.m > 32 && burst(false)))) r.kid = QGEMM_KID_BURST;
            else {
                r.kid = QGEMM_KID_QUAD;
                r.bp = qg::BurstPlan{};
                r.ws_bytes = 0;
                if (have_ws) {
                    r.qsplit = plan_quad_split(x, cus);
                    if (r.qsplit > 1) r.ws_bytes = (size_t)r.qsplit * x.m * x.n * 4;
                }
            }
            return r;
        }
        case QGEMM_KID_TILE256:
            r.kid = kid;
            r.ok = true;
            return r;
        case QGEMM_KID_QUAD:
            r.kid = kid;
            r.ok = x.grid_blocks == 0;    // one tile per workgroup
            return r;
        case QGEMM_KID_BURST:
            r.kid = kid;
            r.ok = x.grid_blocks == 0 && burst(false);
            return r;
        case QGEMM_KID_SLICE:
            r.kid = kid;
            r.sl = plan_slice(x.m, x.n, kt, x.batch, have_ws);
            r.ok = x.grid_blocks == 0 && r.sl.ok;
            r.ws_bytes = r.sl.ws_bytes;
            return r;
        default:
            return r;
    }
}

// Validation of the aiter-format MXFP4 operands (MX4 candidate_m10
// gemm_a4w4_mxfp4_4wave_host.cc:194-250); fills the shared argument block.
hipError_t validate_mx4s(const opus_gemm_mxfp4_scale_kargs* args, int out_dtype, opus_gemm_scale_kargs* common,
                         Spans* sp) {
    if (!args || !args->ptr_a || !args->ptr_b || !args->ptr_c || !args->ptr_sfa || !args->ptr_sfb ||
        !flag01(out_dtype) || args->grid_blocks < 0)
        return hipErrorInvalidValue;
    const auto& x = *args;
    if (x.m <= 0 || x.n <= 0 || x.k <= 0 || x.batch <= 0 || x.k % 256 || x.n % 16) return hipErrorInvalidValue;
    const int kb = x.k / 2, rows32a = ceil_div(x.m, 32), rows32b = ceil_div(x.n, 32);
    // e8m0_shuffle blocks: 32 rows x K/32 groups (K % 256 == 0: no group padding)
    if (x.stride_a < kb || x.stride_b != kb || x.stride_c < x.n || x.stride_sfa < x.k || x.stride_sfb < x.k)
        return hipErrorInvalidValue;
    if (!aligned(x.ptr_a, 16) || !aligned(x.ptr_b, 16) || !aligned(x.ptr_sfa, 16) || !aligned(x.ptr_sfb, 16) ||
        x.stride_a % 16 || x.stride_sfa % 16 || x.stride_sfb % 16)
        return hipErrorInvalidValue;
    const long long outb = out_dtype ? 2 : 4;
    if (!aligned(x.ptr_c, (uintptr_t)outb)) return hipErrorInvalidValue;
    if (x.batch > 1 &&
        ((long long)x.stride_a_batch < (long long)x.m * x.stride_a || x.stride_a_batch % 16 ||
         (long long)x.stride_b_batch < (long long)x.n * kb || x.stride_b_batch % 16 ||
         (long long)x.stride_c_batch < (long long)x.m * x.stride_c ||
         (long long)x.stride_sfa_batch < (long long)rows32a * x.stride_sfa || x.stride_sfa_batch % 16 ||
         (long long)x.stride_sfb_batch < (long long)rows32b * x.stride_sfb || x.stride_sfb_batch % 16))
        return hipErrorInvalidValue;
    if (!bounded_count(x.m, x.stride_a, 1, 1) || !bounded_count(x.n, kb, 1, 1) ||
        !bounded_count(x.m, x.stride_c, 1, outb) || !bounded_count(rows32a, x.stride_sfa, 1, 1) ||
        !bounded_count(rows32b, x.stride_sfb, 1, 1))
        return hipErrorInvalidValue;
    sp->add(x.ptr_c, span(x.batch, x.stride_c_batch, x.m, x.stride_c, x.n, outb));
    sp->add(x.ptr_a, span(x.batch, x.stride_a_batch, x.m, x.stride_a, kb, 1));
    sp->add(x.ptr_b, span(x.batch, x.stride_b_batch, 1, 0, (long long)x.n * kb, 1));
    sp->add(x.ptr_sfa, span(x.batch, x.stride_sfa_batch, rows32a, x.stride_sfa, x.k, 1));
    sp->add(x.ptr_sfb, span(x.batch, x.stride_sfb_batch, rows32b, x.stride_sfb, x.k, 1));
    if (sp->overlap_any(sp->p[0], sp->bytes[0], 1)) return hipErrorInvalidValue;
    std::memcpy(common, &x, sizeof(*common));    // the leading 96 bytes are the common block
    return hipSuccess;
}

}  // namespace

extern "C" {

hipError_t gemm_a4w4_mxfp4_bpreshuffle_kid(const opus_gemm_mxfp4_scale_kargs* args, int out_dtype, int kernel_id,
                                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
    qg::trace_reset();
    Spans sp;
    opus_gemm_scale_kargs a{};
    hipError_t st = validate_mx4s(args, out_dtype, &a, &sp);
    if (st != hipSuccess) return st;
    const auto& x = *args;
    const Mx4sRoute r = route_mx4s(x, kernel_id, workspace != nullptr);
    if (!r.ok) return hipErrorInvalidValue;
    st = check_workspace(workspace, workspace_bytes, r.ws_bytes, sp);
    if (st != hipSuccess) return st;
    st = check_arch();
    if (st != hipSuccess) return st;
    const int kb = x.k / 2;
    const bool bf16 = out_dtype == QGEMM_OUT_BF16;
    TileArgs t{};
    fill_common(t, a, kb, bf16 ? 2 : 4);
    t.sfa_sm = x.stride_sfa;
    t.sfb_sn = x.stride_sfb;
    t.sfa_sk = t.sfb_sk = 256;
    switch (r.kid) {
        case QGEMM_KID_QUAD: {
            if (r.qsplit <= 1) return qg::launch_quad_mx4(t, x.batch, true, bf16, stream);
            // K slices as batch entries: A / B / scale offsets of one slice
            // along K, fp32 output into the partial planes
            const int slice_kt = x.k / 256 / r.qsplit;
            TileArgs w = t;
            w.kbytes = slice_kt * 128;
            w.a_batch = w.kbytes;
            w.b_batch = (long long)slice_kt * 2048;    // within each 16-row block
            w.sfa_batch = w.sfb_batch = (long long)slice_kt * 256;
            float* part = static_cast<float*>(workspace);
            w.c = part;
            w.ldc = x.n;
            w.c_batch = (long long)x.m * x.n;
            w.c_vec = x.n % 4 == 0 ? 4 : x.n % 2 == 0 ? 2 : 1;
            st = qg::launch_quad_mx4(w, r.qsplit, true, false, stream);
            if (st != hipSuccess) return st;
            qg::SplitReduceArgs red{};
            red.ws = part;
            red.c = t.c;
            red.m = x.m;
            red.n = x.n;
            red.ldc = t.ldc;
            red.c_vec = t.c_vec;
            red.splitk = r.qsplit;
            red.batch = 1;
            red.c_batch = t.c_batch;
            return qg::launch_splitk_reduce(red, bf16, stream);
        }
        case QGEMM_KID_SLICE: {
            qg::RunsArgs ra{};
            ra.t = t;
            ra.splitk = r.sl.splitk;
            ra.kt_per_split = r.sl.kt_per_split;
            ra.n_tiles = r.sl.n_tiles;
            ra.b_bytes = (long long)x.n * kb;
            if (r.sl.splitk > 1) {
                ra.counters = static_cast<unsigned*>(workspace);
                ra.epoch = next_epoch();
                ra.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kCounterBytes);
            }
            return qg::launch_slice_mx4s(ra, r.sl.mb, x.batch, bf16, stream);
        }
        case QGEMM_KID_BURST: {
            qg::BurstArgs b{};
            b.t = t;
            b.splitk = r.bp.splitk;
            b.kt_per_split = r.bp.kt_per_split;
            b.n_tiles = r.bp.n_tiles;
            b.b_bytes = (long long)x.n * kb;
            if (r.bp.splitk > 1) {
                b.counters = static_cast<unsigned*>(workspace);
                b.epoch = next_epoch();
                b.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kCounterBytes);
            }
            return qg::launch_burst_mx4s(b, r.bp.mb, r.bp.nb, r.bp.waves, x.batch, bf16, stream);
        }
        default: {
            const long long tiles = (long long)t.tiles_m * t.tiles_n * x.batch;
            const int blocks = x.grid_blocks > 0 ? (int)std::min<long long>(x.grid_blocks, tiles) : 0;
            // 4 K-tiles of scales per DMA when they come whole (K % 1024 == 0)
            return qg::launch_wide_mx4_w16s(t, x.batch, bf16, x.k % 1024 == 0 ? 32 : 8, blocks, stream);
        }
    }
}
size_t gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes(const opus_gemm_mxfp4_scale_kargs* args, int kernel_id) {
    if (!args || args->m <= 0 || args->n <= 0 || args->k <= 0 || args->k % 256 || args->batch <= 0) return 0;
    const Mx4sRoute r = route_mx4s(*args, kernel_id, true);
    return r.ok ? r.ws_bytes : 0;
}
hipError_t gemm_a4w4_mxfp4_bpreshuffle(const opus_gemm_mxfp4_scale_kargs* args, int out_dtype, hipStream_t stream) {
    return gemm_a4w4_mxfp4_bpreshuffle_kid(args, out_dtype, QGEMM_KID_AUTO, nullptr, 0, stream);
}

}  // extern "C"

namespace {

// Scratch memory of gemm_a4w4_mxfp4_noalloc: split-K counters and fp32
// partials, or the wide kernel's panel-major scale copy -- what a caller
// otherwise passes as `workspace`.  Each GPU the library runs on holds its
// own copy of this array until the process ends.  Host code must never pass
// `scratch` itself to a kernel or a copy (on the host it is only a stand-in
// symbol): scratch_ptr() returns this device's address of it.
constexpr size_t kScratchBytes = 32u << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::atomic<uint8_t*> g_scratch_ptr[kMaxDevices];

__global__ void zero_words_kernel(unsigned* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// This device's address of `scratch`, looked up (hipGetSymbolAddress, with the
// device current) on the first call on each device; that call also zeroes the
// split-K counter block on `stream` (a kernel, not a memset, so that the
// first call may be captured into a HIP graph).  Later calls find the
// counters zero again: every split-K launch re-arms the counters it used.
hipError_t scratch_ptr(hipStream_t stream, uint8_t** out) {
    int dev = 0;
    hipError_t st = hipGetDevice(&dev);
    if (st != hipSuccess) return st;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    uint8_t* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* addr = nullptr;
            st = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (st != hipSuccess) return st;
            p = static_cast<uint8_t*>(addr);
            zero_words_kernel<<<1, 256, 0, stream>>>(reinterpret_cast<unsigned*>(p),
                                                     (int)(kCounterBytes / sizeof(unsigned)));
            st = hipGetLastError();
            if (st != hipSuccess) return st;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

}  // namespace

extern "C" {

size_t gemm_a4w4_mxfp4_noalloc_max_workspace_bytes(void) { return kScratchBytes; }

// gemm_a4w4_mxfp4 with the library's static per-device scratch as its
// workspace: no allocation and no caller buffer beyond A, B, scales and C.
// The plan is the one gemm_a4w4_mxfp4 runs with the queried workspace (the
// query is planned without a cap): a call whose query exceeds the scratch is
// refused rather than planned onto another kernel, whose rounding could
// differ.  With need <= kScratchBytes the routes below plan the same: the
// only workspace-dependent choice, the four-wave K split, is taken exactly
// when its bytes fit, and they are part of `need`.
hipError_t gemm_a4w4_mxfp4_noalloc(const opus_gemm_scale_kargs* args, int out_dtype, hipStream_t stream) {
    qg::trace_reset();
    const size_t need = mx_workspace(args, true, QGEMM_KID_AUTO);
    if (need > kScratchBytes) return hipErrorInvalidValue;    // beyond the static scratch
    Spans sp;
    hipError_t st = validate_mx(args, out_dtype, args ? args->k / 2 : 0, 256, &sp);
    if (st != hipSuccess) return st;
    st = check_arch();
    if (st != hipSuccess) return st;
    uint8_t* ws = nullptr;
    st = scratch_ptr(stream, &ws);
    if (st != hipSuccess) return st;
    return gemm_a4w4_mxfp4(args, out_dtype, need ? ws : nullptr, need ? kScratchBytes : 0, stream);
}

// ------------------------------------------------ block-scale FP8, E8M0 scales
// Same checks, in the same order, as SNAP gemm_a8w8_blockscale_bpreshuffle_launch.cc:31-65.
hipError_t launch_blockscale_bpreshuffle(const opus_gemm_scale_kargs* args, int output_bf16, int tiles,
                                         hipStream_t stream) {
    qg::trace_reset();
    if (!args || !args->ptr_a || !args->ptr_b || !args->ptr_c || !args->ptr_sfa || !args->ptr_sfb ||
        !flag01(output_bf16) || !flag01(tiles))
        return hipErrorInvalidValue;
    const auto& a = *args;
    if (a.m <= 0 || a.n <= 0 || a.k <= 0 || a.batch <= 0 || a.m % 256 || a.n % 256 || a.k % 128 ||
        !bounded_count(a.m, a.k, a.batch, 1) || !bounded_count(a.n, a.k, a.batch, 1) ||
        !bounded_count(a.m, a.n, a.batch, output_bf16 ? 2 : 4) || !bounded_count(a.m, a.k / 128, a.batch, 1) ||
        !bounded_count(a.n / 128, a.k / 128, a.batch, 1))
        return hipErrorInvalidValue;
    if (a.stride_a != a.k || a.stride_b != a.k || a.stride_c != a.n || a.stride_a_batch != a.m * a.k ||
        a.stride_b_batch != a.n * a.k || a.stride_c_batch != a.m * a.n || a.stride_sfa != a.m ||
        a.stride_sfb != a.k / 128 || a.stride_sfa_batch != a.m * (a.k / 128) ||
        a.stride_sfb_batch != (a.n / 128) * (a.k / 128))
        return hipErrorInvalidValue;
    const uint64_t c_bytes = uint64_t(a.m) * a.n * a.batch * (output_bf16 ? 2 : 4);
    if (overlaps(a.ptr_c, c_bytes, a.ptr_a, uint64_t(a.stride_a_batch) * a.batch) ||
        overlaps(a.ptr_c, c_bytes, a.ptr_b, uint64_t(a.stride_b_batch) * a.batch) ||
        overlaps(a.ptr_c, c_bytes, a.ptr_sfa, uint64_t(a.stride_sfa_batch) * a.batch) ||
        overlaps(a.ptr_c, c_bytes, a.ptr_sfb, uint64_t(a.stride_sfb_batch) * a.batch))
        return hipErrorInvalidValue;
    if (!dma_aligned(a, false) || !aligned(a.ptr_c, output_bf16 ? 2 : 4)) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    TileArgs t{};
    fill_common(t, a, a.k, output_bf16 ? 2 : 4);
    t.sfa_sk = a.stride_sfa;
    t.sfb_sn = a.stride_sfb;
    return qg::launch_wide_bs8_w16(t, a.batch, output_bf16 == 1, stream);
}

// ------------------------------------------------ E8M0 block scales, NN / TT / TN
// The four-wave tile kernel reads M- or N-contiguous operands as they lie:
// K-major LDS stages, transposed by ds_read_b64_tr_b8 into the same MFMA
// operands as the NT path (TT keeps its row-major [N][K] B).  No workspace.
size_t gemm_a8w8_blockscale_layout_workspace_bytes(const opus_gemm_scale_kargs*, int) { return 0; }

hipError_t gemm_a8w8_blockscale_layout(const opus_gemm_scale_kargs* args, int layout, int output_bf16,
                                       void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (layout == QGEMM_LAYOUT_NT) return launch_blockscale_bpreshuffle(args, output_bf16, 0, stream);
    qg::trace_reset();
    if (!args || !args->ptr_a || !args->ptr_b || !args->ptr_c || !args->ptr_sfa || !args->ptr_sfb ||
        !flag01(output_bf16) || layout < 0 || layout > 3)
        return hipErrorInvalidValue;
    const auto& a = *args;
    const bool at = layout == QGEMM_LAYOUT_TT || layout == QGEMM_LAYOUT_TN;
    const bool bn = layout == QGEMM_LAYOUT_NN || layout == QGEMM_LAYOUT_TN;
    if (a.m <= 0 || a.n <= 0 || a.k <= 0 || a.batch <= 0 || a.m % 256 || a.n % 256 || a.k % 128 ||
        !bounded_count(a.m, a.k, a.batch, 1) || !bounded_count(a.n, a.k, a.batch, 1) ||
        !bounded_count(a.m, a.n, a.batch, output_bf16 ? 2 : 4) || !bounded_count(a.m, a.k / 128, a.batch, 1) ||
        !bounded_count(a.n / 128, a.k / 128, a.batch, 1))
        return hipErrorInvalidValue;
    if (a.stride_a != (at ? a.m : a.k) || a.stride_b != (bn ? a.n : a.k) || a.stride_c != a.n ||
        a.stride_a_batch != a.m * a.k || a.stride_b_batch != a.n * a.k || a.stride_c_batch != a.m * a.n ||
        a.stride_sfa != a.m || a.stride_sfb != a.k / 128 || a.stride_sfa_batch != a.m * (a.k / 128) ||
        a.stride_sfb_batch != (a.n / 128) * (a.k / 128))
        return hipErrorInvalidValue;
    if (!dma_aligned(a, false) || !aligned(a.ptr_c, output_bf16 ? 2 : 4)) return hipErrorInvalidValue;
    Spans sp;
    sp.add(a.ptr_c, uint64_t(a.m) * a.n * a.batch * (output_bf16 ? 2 : 4));
    sp.add(a.ptr_a, uint64_t(a.stride_a_batch) * a.batch);
    sp.add(a.ptr_b, uint64_t(a.stride_b_batch) * a.batch);
    sp.add(a.ptr_sfa, uint64_t(a.stride_sfa_batch) * a.batch);
    sp.add(a.ptr_sfb, uint64_t(a.stride_sfb_batch) * a.batch);
    if (sp.overlap_any(sp.p[0], sp.bytes[0], 1)) return hipErrorInvalidValue;
    (void)workspace;
    (void)workspace_bytes;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    TileArgs t{};
    fill_common(t, a, a.k, output_bf16 ? 2 : 4);
    t.sfa_sk = a.stride_sfa;
    t.sfb_sn = a.stride_sfb;
    return qg::launch_wide_bs8_kmajor(t, a.batch, output_bf16 == 1, at, bn, stream);
}

// ------------------------------------------------ block-scale FP8, fp32 scales
hipError_t gemm_a8w8_blockscale_bpreshuffle_kid(const opus_gemm_kargs* args, int out_dtype, int kernel_id,
                                                void* workspace, size_t workspace_bytes, hipStream_t stream) {
    qg::trace_reset();
    if (!args) return hipErrorInvalidValue;
    const auto& a = *args;
    // B is K-panel [K/128][N][128] (stride_b = 128, BPS host.cc:263)
    if (a.stride_b != 128) return hipErrorInvalidValue;
    const long long bk = (long long)a.n * a.k;
    int sfa_sm = 0, sfa_sk = 0;
    Spans sp;
    hipError_t st = validate_bsf32(a, a.ptr_b, bk, out_dtype, &sfa_sm, &sfa_sk, &sp);
    if (st != hipSuccess) return st;
    if (a.batch > 1 && ((long long)a.stride_b_batch < bk || a.stride_b_batch % 16)) return hipErrorInvalidValue;
    sp.add(a.ptr_b, span(a.batch, a.stride_b_batch, 1, 0, bk, 1));
    if (sp.overlap_any(sp.p[0], sp.bytes[0], sp.n - 1)) return hipErrorInvalidValue;
    const BsfRoute r = route_bsf32(a.m, a.n, a.k / 128, a.batch, bk, false, kernel_id, workspace != nullptr);
    if (!r.ok) return hipErrorInvalidValue;
    st = check_workspace(workspace, workspace_bytes, r.ws_bytes, sp);
    if (st != hipSuccess) return st;
    st = check_arch();
    if (st != hipSuccess) return st;
    TileArgs t{};
    fill_common(t, a, a.k, out_dtype ? 2 : 4);
    t.sfa_sm = sfa_sm;
    t.sfa_sk = sfa_sk;
    t.sfb_sn = a.stride_sfb;
    return run_bsf32(r, t, a.batch, false, bk, out_dtype == QGEMM_OUT_BF16, workspace, workspace_bytes, a.k / 128,
                     stream);
}

size_t gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes(const opus_gemm_kargs* args, int kernel_id) {
    if (!args || args->k <= 0 || args->k % 128) return 0;
    const BsfRoute r = route_bsf32(args->m, args->n, args->k / 128, args->batch, (long long)args->n * args->k, false,
                                   kernel_id, true);
    return r.ok ? r.ws_bytes : 0;
}

hipError_t gemm_a8w8_blockscale_bpreshuffle(const opus_gemm_kargs* args, int out_dtype, void* workspace,
                                            size_t workspace_bytes, hipStream_t stream) {
    return gemm_a8w8_blockscale_bpreshuffle_kid(args, out_dtype, QGEMM_KID_AUTO, workspace, workspace_bytes, stream);
}

size_t gemm_a8w8_blockscale_bpreshuffle_workspace_bytes(const opus_gemm_kargs* args) {
    return gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes(args, QGEMM_KID_AUTO);
}

// ------------------------------------------------ LDS-bypass block-scale FP8
hipError_t gemm_a8w8_blockscale_ldsbypass_kid(const opus_gemm_ldsbypass_kargs* args, int out_dtype, int kernel_id,
                                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
    qg::trace_reset();
    if (!args) return hipErrorInvalidValue;
    const opus_gemm_scale_kargs a = from_ldsbypass(*args);
    const long long bpp = a.n > 0 && a.k > 0 ? (long long)frag_bytes(a.n, a.k) : 0;
    int sfa_sm = 0, sfa_sk = 0;
    Spans sp;
    hipError_t st = validate_bsf32(a, args->ptr_b_pp, bpp, out_dtype, &sfa_sm, &sfa_sk, &sp);
    if (st != hipSuccess) return st;
    if (a.batch > 1 && ((long long)args->stride_b_pp_batch < bpp || args->stride_b_pp_batch % 16))
        return hipErrorInvalidValue;
    sp.add(args->ptr_b_pp, span(a.batch, args->stride_b_pp_batch, 1, 0, bpp, 1));
    if (sp.overlap_any(sp.p[0], sp.bytes[0], sp.n - 1)) return hipErrorInvalidValue;
    // decode shapes: the burst kernel (B'' fragments straight into
    // registers); other small M: the skinny kernel streams B'' into
    // registers; large M: the tile kernels stage B'' blocks through LDS
    const BsfRoute r = route_bsf32(a.m, a.n, a.k / 128, a.batch, bpp, true, kernel_id, workspace != nullptr);
    if (!r.ok) return hipErrorInvalidValue;
    st = check_workspace(workspace, workspace_bytes, r.ws_bytes, sp);
    if (st != hipSuccess) return st;
    st = check_arch();
    if (st != hipSuccess) return st;
    TileArgs t{};
    fill_common(t, a, a.k, out_dtype ? 2 : 4);
    t.sfa_sm = sfa_sm;
    t.sfa_sk = sfa_sk;
    t.sfb_sn = a.stride_sfb;
    return run_bsf32(r, t, a.batch, true, bpp, out_dtype == QGEMM_OUT_BF16, workspace, workspace_bytes, a.k / 128,
                     stream);
}

size_t gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes(const opus_gemm_ldsbypass_kargs* args, int kernel_id) {
    if (!args || args->k <= 0 || args->k % 128 || args->n <= 0) return 0;
    const BsfRoute r = route_bsf32(args->m, args->n, args->k / 128, args->batch,
                                   (long long)frag_bytes(args->n, args->k), true, kernel_id, true);
    return r.ok ? r.ws_bytes : 0;
}

hipError_t gemm_a8w8_blockscale_ldsbypass(const opus_gemm_ldsbypass_kargs* args, int out_dtype, void* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
    return gemm_a8w8_blockscale_ldsbypass_kid(args, out_dtype, QGEMM_KID_AUTO, workspace, workspace_bytes, stream);
}

size_t gemm_a8w8_blockscale_ldsbypass_workspace_bytes(const opus_gemm_ldsbypass_kargs* args) {
    return gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes(args, QGEMM_KID_AUTO);
}

// B' (K-panel, ptr_b, stride_b = 128) -> B'' (ptr_b_pp) on the GPU.
hipError_t gemm_a8w8_blockscale_ldsbypass_repack(const opus_gemm_ldsbypass_kargs* args, hipStream_t stream) {
    qg::trace_reset();
    if (!args || !args->ptr_b || !args->ptr_b_pp) return hipErrorInvalidValue;
    const auto& l = *args;
    if (l.n <= 0 || l.k <= 0 || l.k % 128 || l.batch <= 0 || l.stride_b != 128) return hipErrorInvalidValue;
    const long long bk = (long long)l.n * l.k, bpp = (long long)frag_bytes(l.n, l.k);
    if (!bounded_count(bpp, 1, 1, 1) || !aligned(l.ptr_b, 16) || !aligned(l.ptr_b_pp, 16))
        return hipErrorInvalidValue;
    if (l.batch > 1 &&
        (l.stride_b_batch < bk || l.stride_b_pp_batch < bpp || l.stride_b_batch % 16 || l.stride_b_pp_batch % 16))
        return hipErrorInvalidValue;
    if (overlaps(l.ptr_b, span(l.batch, l.stride_b_batch, 1, 0, bk, 1), l.ptr_b_pp,
                 span(l.batch, l.stride_b_pp_batch, 1, 0, bpp, 1)))
        return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_repack_frag(static_cast<const uint8_t*>(l.ptr_b),
                                  static_cast<uint8_t*>(const_cast<void*>(l.ptr_b_pp)), l.n, l.k, l.batch,
                                  l.stride_b_batch, l.stride_b_pp_batch, stream);
}

// ---------------------------------------------------------------- layouts
int qgemm_shuffle_b_kpanel(const uint8_t* src, uint8_t* dst, int n, int k_bytes) {
    if (!src || !dst || n <= 0 || k_bytes <= 0 || k_bytes % 128) return (int)hipErrorInvalidValue;
    const int nkt = k_bytes / 128;
    for (int r = 0; r < n; ++r)
        for (int kt = 0; kt < nkt; ++kt)
            std::memcpy(dst + ((size_t)kt * n + r) * 128, src + (size_t)r * k_bytes + (size_t)kt * 128, 128);
    return 0;
}

int qgemm_shuffle_weight_16x16(const uint8_t* src, uint8_t* dst, int n, int k_bytes) {
    if (!src || !dst || n <= 0 || k_bytes <= 0 || n % 16 || k_bytes % 16) return (int)hipErrorInvalidValue;
    const int kb = k_bytes / 16;
    for (int b = 0; b < n / 16; ++b)
        for (int c = 0; c < kb; ++c)
            for (int ni = 0; ni < 16; ++ni)
                std::memcpy(dst + ((size_t)b * kb + c) * 256 + (size_t)ni * 16,
                            src + (size_t)(b * 16 + ni) * k_bytes + (size_t)c * 16, 16);
    return 0;
}

size_t qgemm_e8m0_shuffle_bytes(int rows, int groups_k) {
    if (rows <= 0 || groups_k <= 0) return 0;
    return ((size_t)rows + 31) / 32 * 32 * (((size_t)groups_k + 7) / 8 * 8);
}

int qgemm_e8m0_shuffle(const uint8_t* src, uint8_t* dst, int rows, int groups_k) {
    if (!src || !dst || rows <= 0 || groups_k <= 0) return (int)hipErrorInvalidValue;
    const size_t kb8 = ((size_t)groups_k + 7) / 8;    // 8-group blocks per 32-row block
    std::memset(dst, 0x7F, qgemm_e8m0_shuffle_bytes(rows, groups_k));
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < groups_k; ++g) {
            const size_t o = ((size_t)(r / 32) * kb8 + g / 8) * 256 + (size_t)(g % 4) * 64 +
                             (size_t)(r % 16) * 4 + (size_t)((g % 8) / 4) * 2 + (size_t)((r % 32) / 16);
            dst[o] = src[(size_t)r * groups_k + g];
        }
    return 0;
}

size_t qgemm_ldsbypass_b_bytes(int n, int k) {
    if (n <= 0 || k <= 0 || k % 128) return 0;
    return frag_bytes(n, k);
}

// B'' = [ceil(N/16)][K/128][h][lane][16]: lane = 16q + r holds row 16nb + r,
// 16-byte chunk q (h = 0) or q + 4 (h = 1) of the 128-byte K-tile; rows
// past N are zero.
int qgemm_pack_b_ldsbypass(const uint8_t* b_raw, uint8_t* b_pp, int n, int k) {
    if (!b_raw || !b_pp || n <= 0 || k <= 0 || k % 128) return (int)hipErrorInvalidValue;
    const int nk = k / 128, nblk = ceil_div(n, 16);
    for (int nb = 0; nb < nblk; ++nb)
        for (int kt = 0; kt < nk; ++kt)
            for (int h = 0; h < 2; ++h)
                for (int lane = 0; lane < 64; ++lane) {
                    const int row = nb * 16 + (lane & 15), c = (lane >> 4) + 4 * h;
                    uint8_t* d = b_pp + ((((size_t)nb * nk + kt) * 2 + h) * 64 + lane) * 16;
                    if (row < n) std::memcpy(d, b_raw + (size_t)row * k + (size_t)kt * 128 + (size_t)c * 16, 16);
                    else std::memset(d, 0, 16);
                }
    return 0;
}

// ---------------------------------------------------------------- quantizers
}  // extern "C"

namespace {

// Source of a quantizer: fp32 or bf16 rows of at least k elements, pitch a
// multiple of 4 elements and the base aligned for 4-element vector loads.
bool quant_src_ok(const void* x, int in_dtype, int rows, int k, int ldx, int k_align) {
    if (!x || !flag01(in_dtype) || rows <= 0 || k <= 0 || k % k_align || ldx < k || ldx % 4) return false;
    return aligned(x, in_dtype ? 8 : 16);
}

uint64_t src_bytes(int rows, int ldx, int k, int in_dtype) {
    return ((uint64_t)(rows - 1) * ldx + k) * (in_dtype ? 2 : 4);
}

}  // namespace

extern "C" {

hipError_t qgemm_quant_fp8_blockscale_act(const void* x, int in_dtype, int m, int k, int ldx, uint8_t* q, int ldq,
                                          float* scale, int scale_sm, int scale_sk, hipStream_t stream) {
    qg::trace_reset();
    if (!quant_src_ok(x, in_dtype, m, k, ldx, 128) || !q || !scale || ldq < k || ldq % 4 || !aligned(q, 4) ||
        !aligned(scale, 4))
        return hipErrorInvalidValue;
    const int kg = k / 128;
    // scale(m, g) = scale[m*sm + g*sk]: row-major [M][K/128] or column-major [K/128][M]
    if (!((scale_sk == 1 && scale_sm >= kg) || (scale_sm == 1 && scale_sk >= m))) return hipErrorInvalidValue;
    const uint64_t xb = src_bytes(m, ldx, k, in_dtype), qb = (uint64_t)(m - 1) * ldq + k;
    const uint64_t sb = ((uint64_t)(m - 1) * scale_sm + (uint64_t)(kg - 1) * scale_sk + 1) * 4;
    if (overlaps(x, xb, q, qb) || overlaps(x, xb, scale, sb) || overlaps(q, qb, scale, sb)) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_quant_rows(0, 128, in_dtype == 1, false, x, ldx, q, ldq, scale, scale_sm, scale_sk, m, k, stream);
}

hipError_t qgemm_quant_fp8_blockscale_wgt(const void* w, int in_dtype, int n, int k, int ldw, uint8_t* q, int ldq,
                                          float* scale, int ld_scale, hipStream_t stream) {
    qg::trace_reset();
    if (!quant_src_ok(w, in_dtype, n, k, ldw, 128) || !q || !scale || ldq < k || ldq % 4 || !aligned(q, 4) ||
        !aligned(scale, 4) || ld_scale < k / 128)
        return hipErrorInvalidValue;
    const uint64_t xb = src_bytes(n, ldw, k, in_dtype), qb = (uint64_t)(n - 1) * ldq + k;
    const uint64_t sb = ((uint64_t)(ceil_div(n, 128) - 1) * ld_scale + k / 128) * 4;
    if (overlaps(w, xb, q, qb) || overlaps(w, xb, scale, sb) || overlaps(q, qb, scale, sb)) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_quant_wgt_blocks(0, in_dtype == 1, w, ldw, q, ldq, scale, ld_scale, n, k, stream);
}

hipError_t qgemm_quant_fp8_e8m0_act(const void* x, int in_dtype, int m, int k, int ldx, uint8_t* q, int ldq,
                                    uint8_t* e, int e_sm, int e_sk, hipStream_t stream) {
    qg::trace_reset();
    if (!quant_src_ok(x, in_dtype, m, k, ldx, 128) || !q || !e || ldq < k || ldq % 4 || !aligned(q, 4))
        return hipErrorInvalidValue;
    const int kg = k / 128;
    if (!((e_sk == 1 && e_sm >= kg) || (e_sm == 1 && e_sk >= m))) return hipErrorInvalidValue;
    const uint64_t xb = src_bytes(m, ldx, k, in_dtype), qb = (uint64_t)(m - 1) * ldq + k;
    const uint64_t eb = (uint64_t)(m - 1) * e_sm + (uint64_t)(kg - 1) * e_sk + 1;
    if (overlaps(x, xb, q, qb) || overlaps(x, xb, e, eb) || overlaps(q, qb, e, eb)) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_quant_rows(1, 128, in_dtype == 1, false, x, ldx, q, ldq, e, e_sm, e_sk, m, k, stream);
}

hipError_t qgemm_quant_fp8_e8m0_wgt(const void* w, int in_dtype, int n, int k, int ldw, uint8_t* q, int ldq,
                                    uint8_t* e, int ld_e, hipStream_t stream) {
    qg::trace_reset();
    if (!quant_src_ok(w, in_dtype, n, k, ldw, 128) || !q || !e || ldq < k || ldq % 4 || !aligned(q, 4) ||
        ld_e < k / 128)
        return hipErrorInvalidValue;
    const uint64_t xb = src_bytes(n, ldw, k, in_dtype), qb = (uint64_t)(n - 1) * ldq + k;
    const uint64_t eb = (uint64_t)(ceil_div(n, 128) - 1) * ld_e + k / 128;
    if (overlaps(w, xb, q, qb) || overlaps(w, xb, e, eb) || overlaps(q, qb, e, eb)) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_quant_wgt_blocks(1, in_dtype == 1, w, ldw, q, ldq, e, ld_e, n, k, stream);
}

// MXFP8 / MXFP4 share the checks; fp4 packs two codes per byte
static hipError_t quant_mx(bool fp4, const void* x, int in_dtype, int rows, int k, int ldx, uint8_t* q, int ldq,
                           uint8_t* e, int lde, int shuffle, hipStream_t stream) {
    qg::trace_reset();
    const int qrow = fp4 ? k / 2 : k;
    if (!quant_src_ok(x, in_dtype, rows, k, ldx, 32) || !q || !e || !flag01(shuffle) || ldq < qrow ||
        ldq % (fp4 ? 2 : 4) || !aligned(q, fp4 ? 2 : 4) || (!shuffle && lde < k / 32))
        return hipErrorInvalidValue;
    const uint64_t xb = src_bytes(rows, ldx, k, in_dtype), qb = (uint64_t)(rows - 1) * ldq + qrow;
    const uint64_t eb = shuffle ? qgemm_e8m0_shuffle_bytes(rows, k / 32) : (uint64_t)(rows - 1) * lde + k / 32;
    if (overlaps(x, xb, q, qb) || overlaps(x, xb, e, eb) || overlaps(q, qb, e, eb)) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_quant_rows(fp4 ? 2 : 1, 32, in_dtype == 1, shuffle == 1, x, ldx, q, ldq, e, lde, 1, rows, k,
                                 stream);
}

hipError_t qgemm_quant_mxfp8(const void* x, int in_dtype, int rows, int k, int ldx, uint8_t* q, int ldq, uint8_t* e,
                             int lde, int shuffle, hipStream_t stream) {
    return quant_mx(false, x, in_dtype, rows, k, ldx, q, ldq, e, lde, shuffle, stream);
}

hipError_t qgemm_quant_mxfp4(const void* x, int in_dtype, int rows, int k, int ldx, uint8_t* q, int ldq, uint8_t* e,
                             int lde, int shuffle, hipStream_t stream) {
    return quant_mx(true, x, in_dtype, rows, k, ldx, q, ldq, e, lde, shuffle, stream);
}

// ---------------------------------------------------------------- device layouts
static hipError_t relayout(int layout, const uint8_t* src, uint8_t* dst, int n, int k_bytes, int ld_src,
                           int k_align, hipStream_t stream) {
    qg::trace_reset();
    if (!src || !dst || n <= 0 || k_bytes <= 0 || k_bytes % k_align || ld_src < k_bytes || ld_src % 16 ||
        !aligned(src, 16) || !aligned(dst, 16) || (layout == 1 && n % 16))
        return hipErrorInvalidValue;
    const uint64_t sb = (uint64_t)(n - 1) * ld_src + k_bytes;
    const uint64_t db = layout == 2 ? frag_bytes(n, k_bytes) : (uint64_t)n * k_bytes;
    if (overlaps(src, sb, dst, db)) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_relayout(layout, src, dst, n, k_bytes, ld_src, stream);
}

hipError_t qgemm_shuffle_b_kpanel_device(const uint8_t* src, uint8_t* dst, int n, int k_bytes, int ld_src,
                                         hipStream_t stream) {
    return relayout(0, src, dst, n, k_bytes, ld_src, 128, stream);
}

hipError_t qgemm_shuffle_weight_16x16_device(const uint8_t* src, uint8_t* dst, int n, int k_bytes, int ld_src,
                                             hipStream_t stream) {
    return relayout(1, src, dst, n, k_bytes, ld_src, 16, stream);
}

hipError_t qgemm_pack_b_ldsbypass_device(const uint8_t* b_raw, uint8_t* b_pp, int n, int k, int ld_src,
                                         hipStream_t stream) {
    return relayout(2, b_raw, b_pp, n, k, ld_src, 128, stream);
}

hipError_t qgemm_e8m0_shuffle_device(const uint8_t* src, uint8_t* dst, int rows, int groups_k, int ld_src,
                                     hipStream_t stream) {
    qg::trace_reset();
    if (!src || !dst || rows <= 0 || groups_k <= 0 || ld_src < groups_k) return hipErrorInvalidValue;
    if (overlaps(src, (uint64_t)(rows - 1) * ld_src + groups_k, dst, qgemm_e8m0_shuffle_bytes(rows, groups_k)))
        return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    if (aligned(dst, 16) && aligned(src, 4) && ld_src % 4 == 0) {
        qg::ShuffleArgs sh{};
        sh.src[0] = src;
        sh.dst[0] = dst;
        sh.rows[0] = rows;
        sh.ld[0] = ld_src;
        sh.kg = groups_k;
        sh.units[0] = ceil_div(rows, 32) * ceil_div(ceil_div(groups_k, 8), 16);
        return qg::launch_e8m0_shuffle_blocks(sh, 1, stream);
    }
    return qg::launch_e8m0_shuffle(src, dst, rows, groups_k, ld_src, stream);
}

// ---------------------------------------------------------------- probe
int qgemm_probe_words(void) { return qg::kProbeWords; }

hipError_t qgemm_probe_mfma_layout(int32_t* dev_out, hipStream_t stream) {
    if (!dev_out) return hipErrorInvalidValue;
    hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_probe(dev_out, stream);
}

const char* qgemm_version(void) { return "qgemm gfx950 2"; }

const char* qgemm_last_launch(void) { return qg::g_trace_str(); }

}  // extern "C"

// ---------------------------------------------------------------- grouped decode GEMMs
// Several decode GEMMs -- M <= 64 each, batch 1, each with its own N, K,
// operands, scales and output -- in one launch of the burst kernel's grouped
// form (burst_gemm.hpp, BurstGroup): one grid walks every problem's (tile,
// K slice) items, each problem with the fused last-slice split-K reduce of
// its own counters and partial planes.  This is the persistent scheduling
// across mixed decode batches that the reference plans next to its fused
// split-K reduce (R/opus_gemm_splitk_and_interface_refactor.md:41-45) and
// the persistent tile walk of MX4/MULTITILE_DESIGN.md:78: a narrow-N decode
// GEMM alone fills a fraction of the CUs and pays a launch of its own
// (configs[2] M <= 64 at N = 2112-7168 run at 0.13-0.45 of HBM one by one).
namespace {

struct GroupProblem {
    int m, n, kt;    // kt: K-tiles of 128 bytes of K
};

struct GroupPlan {
    bool ok = false;
    int mb = 1, nb = 2, waves = 8, items = 0;
    int splitk[qg::kGroupMax], kt_per[qg::kGroupMax], n_tiles[qg::kGroupMax];
    size_t ctr_off[qg::kGroupMax], part_off[qg::kGroupMax];
    size_t ws_bytes = 0;
    double cost_us = 1e30;
};

// The burst kernel's cost model (burst_gemm.hpp: ~2.5 us per launch, ~25 ns
// per KB one CU streams, ~3.4 us for a K split's coherent round trips) over
// the whole item list, with the HBM stream as a floor: the longest item
// bounds a launch whose items all run at once, the bytes per CU one whose
// items take several rounds.
constexpr double kGroupHbmBytesPerUs = 6.0e6;

double group_cost(const GroupProblem* p, int count, int nb, const int* splitk, const int* kt_per, int cus) {
    double max_kb = 0, sum_kb = 0, bytes = 0;
    bool split = false;
    for (int j = 0; j < count; ++j) {
        const double tiles = ceil_div(p[j].n, 16 * nb);
        const double kb = (16.0 * nb + p[j].m) * kt_per[j] * 128 / 1024.0;
        max_kb = std::max(max_kb, kb);
        sum_kb += kb * tiles * splitk[j];
        bytes += ((double)p[j].n + p[j].m) * p[j].kt * 128;
        split = split || splitk[j] > 1;
    }
    return 2.5 + std::max(0.025 * std::max(max_kb, sum_kb / cus), bytes / kGroupHbmBytesPerUs) + (split ? 3.4 : 0.0);
}

// The plan of a grouped launch: one tile shape, wave count and K-tiles per
// wave for every problem (the kernel is one instantiation), per problem the
// smallest K split the registers allow, then -- with a workspace -- further
// splits of the problem whose items stream the most bytes while the cost
// model drops by at least 1%.  Workspace: the split problems' counter words
// (one per tile), then each split problem's fp32 partial planes.
GroupPlan plan_grouped(const GroupProblem* p, int count, bool mx, bool frag, int cus, bool allow_split) {
    GroupPlan best;
    if (count < 1 || count > qg::kGroupMax) return best;
    int mmax = 0;
    for (int j = 0; j < count; ++j) {
        if (p[j].m < 1 || p[j].m > 64 || p[j].n < 1 || p[j].kt < 1) return best;
        mmax = std::max(mmax, p[j].m);
    }
    const int mb = mmax <= 16 ? 1 : (mmax <= 32 ? 2 : 4);
    // 16 waves first: on a tie (the same items and bytes) the plan that puts
    // twice the waves' loads in flight per item wins -- configs[2]'s decode
    // trio, fp32 block scales, M = 1 / 16: 18.3 / 21.1 us with 8 waves x 8
    // K-tiles, 17.5 / 19.2 us with 16 x 4
    for (int nb : {2, 1})
        for (int waves : {16, 8}) {
            const int kmax = qg::burst_max_kpw(mb, nb, waves, mx);
            if (kmax == 0 || qg::burst_lds_bytes(mb, nb, waves, !frag) > qg::kBurstLdsMax) continue;
            const int cap = waves * kmax;
            GroupPlan c;
            c.mb = mb;
            c.nb = nb;
            c.waves = waves;
            bool ok = true;
            auto can_split = [&](int j) { return allow_split && (long long)p[j].m * p[j].n < (1LL << 29); };
            for (int j = 0; j < count && ok; ++j) {
                int s = ceil_div(p[j].kt, cap);
                const int kp = ceil_div(p[j].kt, s);
                s = ceil_div(p[j].kt, kp);
                if (s > 1 && (!can_split(j) || s > kMaxSplit)) ok = false;
                c.splitk[j] = s;
                c.kt_per[j] = kp;
                c.n_tiles[j] = ceil_div(p[j].n, 16 * nb);
            }
            if (!ok) continue;
            c.cost_us = group_cost(p, count, nb, c.splitk, c.kt_per, cus);
            for (int step = 0; step < 64; ++step) {
                int jb = -1;
                double kb_max = 0;
                for (int j = 0; j < count; ++j) {
                    const double kb = (16.0 * nb + p[j].m) * c.kt_per[j];
                    if (can_split(j) && c.kt_per[j] > 1 && c.splitk[j] < kMaxSplit && kb > kb_max) {
                        kb_max = kb;
                        jb = j;
                    }
                }
                if (jb < 0) break;
                const int s0 = c.splitk[jb], k0 = c.kt_per[jb];
                const int kp = ceil_div(p[jb].kt, s0 + 1);
                c.kt_per[jb] = kp;
                c.splitk[jb] = ceil_div(p[jb].kt, kp);
                const double cost = group_cost(p, count, nb, c.splitk, c.kt_per, cus);
                if (cost < 0.99 * c.cost_us) {
                    c.cost_us = cost;
                } else {
                    c.splitk[jb] = s0;
                    c.kt_per[jb] = k0;
                    break;
                }
            }
            if (c.cost_us < best.cost_us) {
                c.ok = true;
                best = c;
            }
        }
    if (!best.ok) return best;
    size_t ctr = 0, part = 0;
    best.items = 0;
    for (int j = 0; j < count; ++j) {
        best.items += best.n_tiles[j] * best.splitk[j];
        best.ctr_off[j] = ctr;
        if (best.splitk[j] > 1) ctr += (size_t)best.n_tiles[j] * sizeof(unsigned);
    }
    ctr = round256(ctr);
    for (int j = 0; j < count; ++j) {
        best.part_off[j] = ctr + part;
        if (best.splitk[j] > 1) part += round256((size_t)best.splitk[j] * p[j].m * p[j].n * sizeof(float));
    }
    best.ws_bytes = part ? ctr + part : 0;
    return best;
}

enum class GroupFam { BS_KPANEL, BS_FRAG, MX8, MX4 };

// A grouped call's problems, validated one by one as their single-problem
// entries do (batch 1, M <= 64 added), as kernel tiles.
struct GroupCall {
    int count = 0;
    qg::TileArgs t[qg::kGroupMax];
    long long b_bytes[qg::kGroupMax];
    GroupProblem shape[qg::kGroupMax];
    const void* span_p[qg::kGroupMax * 6];
    uint64_t span_b[qg::kGroupMax * 6];
    int spans = 0;
};

hipError_t group_problem(GroupFam fam, const void* kargs, int j, int out_dtype, GroupCall* g) {
    opus_gemm_scale_kargs a{};
    const void* b_data = nullptr;
    long long bb = 0;
    Spans sp;
    int sfa_sm = 0, sfa_sk = 0;
    hipError_t st = hipSuccess;
    if (fam == GroupFam::BS_FRAG) {
        const auto& l = static_cast<const opus_gemm_ldsbypass_kargs*>(kargs)[j];
        a = from_ldsbypass(l);
        b_data = l.ptr_b_pp;
        bb = a.n > 0 && a.k > 0 ? (long long)frag_bytes(a.n, a.k) : 0;
    } else {
        a = static_cast<const opus_gemm_scale_kargs*>(kargs)[j];
        b_data = a.ptr_b;
    }
    if (a.batch != 1 || a.m < 1 || a.m > 64) return hipErrorInvalidValue;
    const bool fp4 = fam == GroupFam::MX4;
    const int kbytes = fp4 ? a.k / 2 : a.k;
    if (fam == GroupFam::BS_KPANEL || fam == GroupFam::BS_FRAG) {
        if (fam == GroupFam::BS_KPANEL) {
            if (a.stride_b != 128) return hipErrorInvalidValue;    // K-panel B' (BPS host.cc:263)
            bb = (long long)a.n * a.k;
        }
        st = validate_bsf32(a, b_data, bb, out_dtype, &sfa_sm, &sfa_sk, &sp);
        if (st != hipSuccess) return st;
        sp.add(b_data, (uint64_t)bb);
        if (sp.overlap_any(sp.p[0], sp.bytes[0], sp.n - 1)) return hipErrorInvalidValue;
    } else {
        st = validate_mx(&a, out_dtype, kbytes, fp4 ? 256 : 128, &sp);
        if (st != hipSuccess) return st;
        bb = (long long)(a.n - 1) * a.stride_b + kbytes;
    }
    qg::TileArgs& t = g->t[j];
    t = qg::TileArgs{};
    fill_common(t, a, kbytes, out_dtype ? 2 : 4);
    if (fam == GroupFam::BS_KPANEL || fam == GroupFam::BS_FRAG) {
        t.sfa_sm = sfa_sm;
        t.sfa_sk = sfa_sk;
    } else {
        t.sfa_sm = a.stride_sfa;
    }
    t.sfb_sn = a.stride_sfb;
    g->b_bytes[j] = bb;
    g->shape[j] = GroupProblem{a.m, a.n, kbytes / 128};
    // C first: every problem's output is checked against every operand of the call
    for (int i = 0; i < sp.n; ++i) {
        g->span_p[g->spans] = sp.p[i];
        g->span_b[g->spans++] = sp.bytes[i];
    }
    return hipSuccess;
}

hipError_t group_collect(GroupFam fam, const void* kargs, int count, int out_dtype, GroupCall* g,
                         int* span_begin) {
    if (!kargs || count < 1 || count > qg::kGroupMax || !flag01(out_dtype)) return hipErrorInvalidValue;
    g->count = count;
    for (int j = 0; j < count; ++j) {
        span_begin[j] = g->spans;
        const hipError_t st = group_problem(fam, kargs, j, out_dtype, g);
        if (st != hipSuccess) return st;
    }
    span_begin[count] = g->spans;
    // outputs may not overlap any other problem's operands or outputs
    for (int j = 0; j < count; ++j) {
        const void* c = g->span_p[span_begin[j]];
        const uint64_t cb = g->span_b[span_begin[j]];
        for (int i = 0; i < g->spans; ++i)
            if ((i < span_begin[j] || i >= span_begin[j + 1]) && overlaps(c, cb, g->span_p[i], g->span_b[i]))
                return hipErrorInvalidValue;
    }
    return hipSuccess;
}

GroupPlan group_plan(GroupFam fam, const GroupCall& g, bool allow_split) {
    return plan_grouped(g.shape, g.count, fam == GroupFam::MX8 || fam == GroupFam::MX4, fam == GroupFam::BS_FRAG,
                        device_cus(), allow_split);
}

hipError_t group_entry(GroupFam fam, const void* kargs, int count, int out_dtype, int grid_blocks, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
    qg::trace_reset();
    if (grid_blocks < 0) return hipErrorInvalidValue;
    GroupCall g;
    int span_begin[qg::kGroupMax + 1];
    hipError_t st = group_collect(fam, kargs, count, out_dtype, &g, span_begin);
    if (st != hipSuccess) return st;
    const GroupPlan pl = group_plan(fam, g, ws != nullptr);
    if (!pl.ok) return hipErrorInvalidValue;
    if (ws && pl.ws_bytes) {
        if (ws_bytes < pl.ws_bytes || !aligned(ws, 256)) return hipErrorInvalidValue;
        for (int i = 0; i < g.spans; ++i)
            if (overlaps(ws, pl.ws_bytes, g.span_p[i], g.span_b[i])) return hipErrorInvalidValue;
    }
    st = check_arch();
    if (st != hipSuccess) return st;
    qg::BurstGroup bg{};
    bg.count = count;
    const unsigned epoch = next_epoch();
    int item = 0;
    for (int j = 0; j < count; ++j) {
        qg::BurstArgs& b = bg.p[j];
        b.t = g.t[j];
        b.splitk = pl.splitk[j];
        b.kt_per_split = pl.kt_per[j];
        b.n_tiles = pl.n_tiles[j];
        b.b_bytes = g.b_bytes[j];
        b.epoch = epoch;
        if (pl.splitk[j] > 1) {
            b.counters = reinterpret_cast<unsigned*>(static_cast<uint8_t*>(ws) + pl.ctr_off[j]);
            b.ws = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + pl.part_off[j]);
        }
        bg.item_begin[j] = item;
        item += pl.n_tiles[j] * pl.splitk[j];
    }
    bg.item_begin[count] = item;
    const int grid = grid_blocks > 0 ? std::min(grid_blocks, item) : item;
    const bool bf16 = out_dtype == QGEMM_OUT_BF16;
    switch (fam) {
        case GroupFam::BS_KPANEL:
            return qg::launch_burst_grouped(bg, false, pl.mb, pl.nb, pl.waves, grid, bf16, stream);
        case GroupFam::BS_FRAG:
            return qg::launch_burst_grouped(bg, true, pl.mb, pl.nb, pl.waves, grid, bf16, stream);
        case GroupFam::MX8:
            return qg::launch_burst_mx_grouped(bg, false, pl.mb, pl.nb, pl.waves, grid, bf16, stream);
        default:
            return qg::launch_burst_mx_grouped(bg, true, pl.mb, pl.nb, pl.waves, grid, bf16, stream);
    }
}

// The workspace the grouped call's split plan needs (0: no problem splits,
// or the arguments are not a valid grouped call).
size_t group_workspace(GroupFam fam, const void* kargs, int count) {
    GroupCall g;
    int span_begin[qg::kGroupMax + 1];
    if (group_collect(fam, kargs, count, QGEMM_OUT_BF16, &g, span_begin) != hipSuccess) return 0;
    const GroupPlan pl = group_plan(fam, g, true);
    return pl.ok ? pl.ws_bytes : 0;
}

}  // namespace

extern "C" {

hipError_t gemm_a8w8_blockscale_bpreshuffle_grouped(const opus_gemm_kargs* args, int group_count, int out_dtype,
                                                    int grid_blocks, void* workspace, size_t workspace_bytes,
                                                    hipStream_t stream) {
    return group_entry(GroupFam::BS_KPANEL, args, group_count, out_dtype, grid_blocks, workspace, workspace_bytes,
                       stream);
}
size_t gemm_a8w8_blockscale_bpreshuffle_grouped_workspace_bytes(const opus_gemm_kargs* args, int group_count) {
    return group_workspace(GroupFam::BS_KPANEL, args, group_count);
}

hipError_t gemm_a8w8_blockscale_ldsbypass_grouped(const opus_gemm_ldsbypass_kargs* args, int group_count,
                                                  int out_dtype, int grid_blocks, void* workspace,
                                                  size_t workspace_bytes, hipStream_t stream) {
    return group_entry(GroupFam::BS_FRAG, args, group_count, out_dtype, grid_blocks, workspace, workspace_bytes,
                       stream);
}
size_t gemm_a8w8_blockscale_ldsbypass_grouped_workspace_bytes(const opus_gemm_ldsbypass_kargs* args,
                                                              int group_count) {
    return group_workspace(GroupFam::BS_FRAG, args, group_count);
}

hipError_t gemm_a8w8_mxfp8_grouped(const opus_gemm_scale_kargs* args, int group_count, int out_dtype, int grid_blocks,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return group_entry(GroupFam::MX8, args, group_count, out_dtype, grid_blocks, workspace, workspace_bytes, stream);
}
size_t gemm_a8w8_mxfp8_grouped_workspace_bytes(const opus_gemm_scale_kargs* args, int group_count) {
    return group_workspace(GroupFam::MX8, args, group_count);
}

hipError_t gemm_a4w4_mxfp4_grouped(const opus_gemm_scale_kargs* args, int group_count, int out_dtype, int grid_blocks,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return group_entry(GroupFam::MX4, args, group_count, out_dtype, grid_blocks, workspace, workspace_bytes, stream);
}
size_t gemm_a4w4_mxfp4_grouped_workspace_bytes(const opus_gemm_scale_kargs* args, int group_count) {
    return group_workspace(GroupFam::MX4, args, group_count);
}

}  // extern "C"

// ---------------------------------------------------------------- whole-output reference GEMM
extern "C" {

// Validation and launch of ref_gemm.hip (see qgemm.h): batch 1, row-major
// codes, fp32 output that overlaps no input.
hipError_t qgemm_reference_gemm(int family, const opus_gemm_scale_kargs* args, hipStream_t stream) {
    qg::trace_reset();
    if (!args || family < QGEMM_REF_BS_FP32 || family > QGEMM_REF_MXFP4) return hipErrorInvalidValue;
    const auto& a = *args;
    if (!a.ptr_a || !a.ptr_b || !a.ptr_c || !a.ptr_sfa || !a.ptr_sfb || a.batch != 1 || a.m <= 0 || a.n <= 0 ||
        a.k <= 0)
        return hipErrorInvalidValue;
    const bool mx = family == QGEMM_REF_MXFP8 || family == QGEMM_REF_MXFP4;
    const bool fp4 = family == QGEMM_REF_MXFP4;
    if (a.k % (mx ? 32 : 128)) return hipErrorInvalidValue;
    const long long kbytes = fp4 ? a.k / 2 : a.k, kg = a.k / (mx ? 32 : 128), nbk = ceil_div(a.n, 128);
    if (a.stride_a < kbytes || a.stride_b < kbytes || a.stride_c < a.n || !aligned(a.ptr_c, 4))
        return hipErrorInvalidValue;
    qg::RefArgs r{};
    r.a = static_cast<const uint8_t*>(a.ptr_a);
    r.b = static_cast<const uint8_t*>(a.ptr_b);
    r.sfa = static_cast<const uint8_t*>(a.ptr_sfa);
    r.sfb = static_cast<const uint8_t*>(a.ptr_sfb);
    r.c = static_cast<float*>(a.ptr_c);
    r.m = a.m;
    r.n = a.n;
    r.k = a.k;
    r.lda = a.stride_a;
    r.ldb = a.stride_b;
    r.ldc = a.stride_c;
    uint64_t sfa_bytes, sfb_bytes;
    const int elem = family == QGEMM_REF_BS_FP32 ? 4 : 1;
    if (mx) {
        if (a.stride_sfa < kg || a.stride_sfb < kg) return hipErrorInvalidValue;
        r.sfa_sm = a.stride_sfa;
        r.sfb_sm = a.stride_sfb;
        sfa_bytes = (uint64_t)(a.m - 1) * a.stride_sfa + kg;
        sfb_bytes = (uint64_t)(a.n - 1) * a.stride_sfb + kg;
    } else {
        // A's scales: row-major [M][K/128] (stride_sfa = 1, M > 1) or
        // column-major [K/128][M] (stride_sfa >= M), as the product entries
        const bool rowmajor = a.stride_sfa == 1 && a.m > 1;
        if (a.stride_sfb < kg || (!rowmajor && a.stride_sfa < a.m)) return hipErrorInvalidValue;
        if (elem == 4 && (!aligned(a.ptr_sfa, 4) || !aligned(a.ptr_sfb, 4))) return hipErrorInvalidValue;
        r.sfa_sm = rowmajor ? kg : 1;
        r.sfa_sk = rowmajor ? 1 : a.stride_sfa;
        r.sfb_sm = a.stride_sfb;
        sfa_bytes = (rowmajor ? (uint64_t)a.m * kg : (uint64_t)(kg - 1) * a.stride_sfa + a.m) * elem;
        sfb_bytes = ((uint64_t)(nbk - 1) * a.stride_sfb + kg) * elem;
    }
    const uint64_t cb = ((uint64_t)(a.m - 1) * a.stride_c + a.n) * 4;
    if (overlaps(a.ptr_c, cb, a.ptr_a, (uint64_t)(a.m - 1) * a.stride_a + kbytes) ||
        overlaps(a.ptr_c, cb, a.ptr_b, (uint64_t)(a.n - 1) * a.stride_b + kbytes) ||
        overlaps(a.ptr_c, cb, a.ptr_sfa, sfa_bytes) || overlaps(a.ptr_c, cb, a.ptr_sfb, sfb_bytes))
        return hipErrorInvalidValue;
    const hipError_t st = check_arch();
    if (st != hipSuccess) return st;
    return qg::launch_ref_gemm(r, static_cast<qg::RefFam>(family), stream);
}

}  // extern "C"
