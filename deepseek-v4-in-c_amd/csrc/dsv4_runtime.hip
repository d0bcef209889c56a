/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_runtime.hip - the C ABI (include/dsv4_hip.h, include/dsv4_hip_aux.h):
 * device selection, the upload-once weight registry, staging for the
 * host-pointer entry points, and argument checking before any launch.
 *
 * Conventions follow the reference's GPU backend
 * (src/80_prefill/dsv4_prefill_vk.h:31-49, dsv4_prefill_vk_gemm.c:63-132):
 * init returns -1 when no device is usable; a call returns 0 when the GPU
 * produced the whole result and -1 otherwise, leaving the caller's CPU path in
 * charge; a HIP runtime failure latches `dead` so every later call returns -1
 * at once. The library is not re-entrant across host threads (one mutex
 * serialises the host-pointer calls, as the Vulkan backend's single command
 * buffer and fence do) and nothing here computes on the CPU.
 *
 * Kernels report bad input through a device status word. Host-pointer calls
 * use a word of their own, read after the call's synchronisation: any bit
 * turns the call into -1, so 0 always means the GPU produced the whole
 * result. _dev calls use another word, read with dsv4_hip_status().
 *
 * DSV4_HIP_DISABLE=1 in the environment makes dsv4_hip_init() fail, which
 * forces every caller onto its CPU path (the reference's behaviour on a
 * machine without the GPU backend). Every entry point is one roctx range
 * named after it, visible in rocprofv3 --marker-trace.
 */
#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include <algorithm>

#include <dirent.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdlib.h>
#include <unistd.h>
#include <stdio.h>
#include <string.h>

#include <rocprofiler-sdk-roctx/roctx.h>

#include "dsv4_internal.h"
#include "../../include/dsv4_hip_aux.h"

using namespace dsv4;

namespace {

struct Region {
    size_t bytes;
    void *dev;
};

/* Every device allocation of the library goes through dev_malloc, which
 * counts the attempts (dsv4_hip_alloc_count). */
std::atomic<unsigned long long> g_alloc_calls{0};
hipError_t dev_malloc(void **p, size_t bytes)
{
    g_alloc_calls.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(p, bytes);
}

/* A device buffer that only grows. */
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    hipError_t need(size_t bytes)
    {
        if (bytes <= cap) return hipSuccess;
        if (p) { (void)hipFree(p); p = nullptr; cap = 0; }
        const size_t want = bytes < 4096 ? 4096 : bytes;
        hipError_t e = dev_malloc(&p, want);
        if (e == hipSuccess) cap = want;
        return e;
    }
    void release()
    {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

struct State {
    std::mutex mu;
    int ready = 0;
    int dead = 0;
    int device = -1;
    hipStream_t stream = nullptr;
    hipStream_t side = nullptr;          /* concurrent work of one call (shared expert) */
    hipStream_t side2 = nullptr;         /* concurrent work of one call (thin routed tiles) */
    hipEvent_t fork = nullptr, join = nullptr, fork2 = nullptr, join2 = nullptr, xq = nullptr;
    unsigned *status = nullptr;          /* status words: [0] _dev calls, [HOST_WORD] host calls */
    unsigned *st = nullptr;              /* the word the call being enqueued raises */
    unsigned *pub = nullptr;             /* one-launch decode: count, done, leave (own lines) */
    unsigned *rt_count = nullptr;        /* fused gate + router: arrival counters (zero between launches) */
    std::map<uintptr_t, Region> regions; /* host start -> resident copy   */
    DevBuf x, y, mid, table, small, ys, gemm_ws, moe_ws, x16, msplit, route;
};

constexpr int HOST_WORD = 32;            /* the host calls' word, on its own 128-byte line */

/* Device scratch of dsv4_hip_moe_decode_routed_noalloc_dev, the entry point
 * for callers that cannot allocate: the one-launch hand-off words (zero
 * between launches), the mid rows, the mid split tables and the shared
 * expert's output of one decode MoE call with topk <= 8, inter <= 2048 and
 * hidden <= 4096 (174,592 bytes at those maxima: 2,560 + 9 x 2048 x 4 +
 * 8 x 16 x 640 + 4096 x 4). Each GPU holds its own
 * copy until the process ends. Host code uses only the device address that
 * hipGetSymbolAddress returns for it (scratch_ptr, filled at init), never
 * this name. */
constexpr size_t SCRATCH_BYTES = 174592;
__device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
void *scratch_ptr_of[MAX_DEVICES];       /* device address of `scratch` per device */

State g;
thread_local std::string g_err;

/* One roctx range per entry point call. */
struct Range {
    explicit Range(const char *name) { roctxRangePushA(name); }
    ~Range() { roctxRangePop(); }
};

int fail(const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}

int hip_fail(hipError_t e, const char *what)
{
    g.dead = 1;
    return fail("%s: %s (backend latched dead)", what, hipGetErrorString(e));
}

#define HIPCHK(expr, what)                                                     \
    do {                                                                       \
        hipError_t e_ = (expr);                                                \
        if (e_ != hipSuccess) return hip_fail(e_, what);                       \
    } while (0)

int usable(void)
{
    if (!g.ready) return fail("dsv4_hip_init has not succeeded");
    if (g.dead) return fail("backend is dead after an earlier HIP failure");
    return 0;
}

/* The calls that follow raise the _dev status word or the host calls' word. */
void dev_call(void) { g.st = g.status; }
void host_call(void) { g.st = g.status + HOST_WORD; }

std::string status_text(unsigned v)
{
    static const char *const names[] = {
        "routing id out of range", "expert descriptor of the wrong format",
        "FP4 scale byte outside 104..140 on an fp16 path", "one-launch decode wait timed out",
        "SwiGLU output beyond the fp16 range"};
    std::string s;
    for (unsigned b = 0; b < sizeof names / sizeof names[0]; b++)
        if (v & (1u << b)) s += (s.empty() ? "" : "; ") + std::string(names[b]);
    return s.empty() ? std::string("unknown bits") : s;
}

/* End of a host-pointer call whose work is enqueued on g.stream: wait for it,
 * then read the host calls' status word; any bit makes the call -1 (its
 * output is not the whole, valid result) and is cleared. */
int finish_host_call(const char *what)
{
    unsigned v = 0;
    HIPCHK(hipMemcpyAsync(&v, g.status + HOST_WORD, sizeof v, hipMemcpyDeviceToHost, g.stream),
           "status read");
    HIPCHK(hipStreamSynchronize(g.stream), what);
    if (v) {
        HIPCHK(hipMemsetAsync(g.status + HOST_WORD, 0, sizeof v, g.stream), "status clear");
        HIPCHK(hipStreamSynchronize(g.stream), "status clear");
        return fail("%s: the device raised status 0x%x (%s)", what, v, status_text(v).c_str());
    }
    return 0;
}

/* Device copy of [p, p + bytes) when it lies inside one registered range. */
const void *translate(const void *p, size_t bytes)
{
    if (!p) return nullptr;
    const uintptr_t a = (uintptr_t)p;
    auto it = g.regions.upper_bound(a);
    if (it == g.regions.begin()) return nullptr;
    --it;
    const uintptr_t s = it->first;
    if (a < s || a + bytes > s + it->second.bytes) return nullptr;
    return (const uint8_t *)it->second.dev + (a - s);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

/* Check a descriptor the GPU path can run and compute its byte sizes. */
/* allow_generic (the matvec entry points): a packed matrix of any other
 * block geometry, or with rows wider than the fast kernels take, gets its
 * FMT_GEN_* format (the generic matvec) instead of a refusal. */
int check_qmat(const DSV4QMat *m, const char *what, int *fmt, bool allow_generic = false)
{
    if (!m) return fail("%s: NULL matrix", what);
    *fmt = qmat_fmt(m);
    if (*fmt < 0 && allow_generic) *fmt = qmat_fmt_generic(m);
    if (*fmt < 0)
        return fail("%s: unsupported geometry wdt=%d %dx%d blk %dx%d", what,
                    m->wdt, m->rows, m->cols, m->blk_r, m->blk_c);
    if (*fmt >= FMT_GEN_FP8) return 0;
    /* FP8 up to 8192 columns, FP4 up to 16384, BF16 up to 8192 */
    const int lim = *fmt == FMT_BF16 ? 16384 : 8192;
    if (qmat_row_bytes(m) > lim) {
        if (allow_generic && *fmt != FMT_BF16) {
            *fmt = qmat_fmt_generic(m);
            return 0;
        }
        return fail("%s: rows wider than %d bytes are not supported", what, lim);
    }
    return 0;
}

/* Host descriptor -> descriptor with resident device pointers (BF16 has no
 * scales). */
int resident(const DSV4QMat *m, DSV4QMat *out, const char *what, bool allow_generic = false,
             int *fmt_out = nullptr)
{
    int fmt;
    if (check_qmat(m, what, &fmt, allow_generic)) return -1;
    if (fmt_out) *fmt_out = fmt;
    *out = *m;
    out->w = translate(m->w, qmat_w_bytes(m));
    out->s = fmt == FMT_BF16 ? nullptr : translate(m->s, qmat_s_bytes(m));
    if (!out->w || (fmt != FMT_BF16 && !out->s))
        return fail("%s: weights or scales are not inside a registered range", what);
    if (!aligned16(out->w)) return fail("%s: weights are not 16-byte aligned", what);
    return 0;
}

int expert_geometry(const DSV4ExpertW *e, int *fmt, int *inter, int *hidden,
                    const char *what)
{
    int f1, f3, f2;
    if (check_qmat(&e->w1, what, &f1) || check_qmat(&e->w3, what, &f3) ||
        check_qmat(&e->w2, what, &f2))
        return -1;
    if (f1 != f3 || f1 != f2) return fail("%s: w1/w3/w2 formats differ", what);
    if (f1 == FMT_BF16) return fail("%s: experts must be FP8 or FP4", what);
    if (e->w1.rows != e->w3.rows || e->w1.cols != e->w3.cols ||
        e->w2.rows != e->w1.cols || e->w2.cols != e->w1.rows)
        return fail("%s: w1/w3/w2 shapes do not chain", what);
    *fmt = f1;
    *inter = e->w1.rows;
    *hidden = e->w1.cols;
    return 0;
}

int resident_expert(const DSV4ExpertW *e, DSV4ExpertW *out, const char *what)
{
    if (resident(&e->w1, &out->w1, what) || resident(&e->w3, &out->w3, what) ||
        resident(&e->w2, &out->w2, what))
        return -1;
    return 0;
}

GemvArgs gemv_args(const DSV4QMat &m, const float *x, float *y, int nt)
{
    GemvArgs a;
    a.W = (const uint8_t *)m.w;
    a.S = m.s;
    a.x = x;
    a.y = y;
    a.rows = m.rows;
    a.row_bytes = qmat_row_bytes(&m);
    a.sc_cols = qmat_sc_cols(&m);
    a.blk_r = m.blk_r;
    a.nt = nt;
    a.x_ld = m.cols;
    a.y_ld = m.rows;
    return a;
}

/* The block-scaled MFMA GEMV takes matrices whose columns are whole 128-wide
 * chunks (at most 8192 FP8 or FP4 columns), FP8 row blocks that are
 * multiples of 16 rows, 4-byte aligned fp32 scales and 16-byte aligned x. */
bool mx_gemv_ok(const DSV4QMat &d, int fmt, const float *x)
{
    if (!gemv_mx_ncw(fmt, d.cols) || !aligned16(x) || !aligned16(d.w)) return false;
    if (fmt != FMT_FP4_E8M0 && d.blk_r % 16) return false;
    if (fmt == FMT_FP8_F32S && ((uintptr_t)d.s & 3u)) return false;
    return true;
}

GemvMxArgs gemv_mx_args(const DSV4QMat &m, const float *x, float *y, int nt)
{
    GemvMxArgs a;
    memset(&a, 0, sizeof a);
    a.W = (const uint8_t *)m.w;
    a.S = m.s;
    a.x = x;
    a.y = y;
    a.rows = m.rows;
    a.cols = m.cols;
    a.row_bytes = qmat_row_bytes(&m);
    a.sc_cols = qmat_sc_cols(&m);
    a.blk_r = m.blk_r;
    a.nt = nt;
    a.x_ld = m.cols;
    a.y_ld = m.rows;
    return a;
}

/* Expert shapes the MFMA gate/up takes: inter and hidden whole 128-wide
 * chunks within the GEMV limits. */
bool mx_expert_ok(int fmt, int inter, int hidden)
{
    return inter > 0 && inter % 128 == 0 && gateup_mx_ncw(fmt, hidden) && gemv_mx_ncw(fmt, inter);
}

/* Enqueue one expert (gate/up + SwiGLU -> mid, then w2 -> out) from a
 * descriptor holding device pointers. */
int enqueue_expert(const DSV4ExpertW &e, int fmt, int inter, int hidden,
                   const float *x, float *mid, float *out, float limit,
                   hipStream_t st)
{
    const bool mx = mx_expert_ok(fmt, inter, hidden) && aligned16(x) && aligned16(mid) &&
                    mx_gemv_ok(e.w2, fmt, mid) &&
                    (fmt != FMT_FP8_F32S || (((uintptr_t)e.w1.s | (uintptr_t)e.w3.s) & 3u) == 0);
    if (mx) {
        GateUpMxArgs ga;
        memset(&ga, 0, sizeof ga);
        ga.direct = e;
        ga.use_direct = 1;
        ga.nslots = 1;
        ga.x = x;
        ga.mid = mid;
        ga.mid_ld = inter;
        ga.inter = inter;
        ga.hidden = hidden;
        ga.limit = limit;
        ga.status = g.st;
        HIPCHK(gateup_mx_launch(fmt, ga, st), "gate/up launch");
        HIPCHK(gemv_mx_launch(fmt, gemv_mx_args(e.w2, mid, out, 1), st), "down launch");
        return 0;
    }
    GateUpArgs ga;
    memset(&ga, 0, sizeof ga);
    ga.direct = e;
    ga.use_direct = 1;
    ga.nslots = 1;
    ga.x = x;
    ga.mid = mid;
    ga.mid_ld = inter;
    ga.inter = inter;
    ga.hidden = hidden;
    ga.limit = limit;
    ga.status = g.st;
    HIPCHK(gateup_launch(fmt, ga, st), "gate/up launch");
    HIPCHK(gemv_launch(fmt, gemv_args(e.w2, mid, out, 1), st), "down launch");
    return 0;
}

/* Device memory of one decode MoE call: the mid rows of the routed slots
 * ([topk][mid_ld]) followed by the shared expert's, the split tables of the
 * routed mids ([topk][mx_split_bytes(inter)]), the shared expert's output
 * [hidden] and the one-launch publication words (ONE_PUB_BYTES, zero between
 * launches). */
struct MoeWs {
    float *mid;
    uint8_t *msplit;          /* split tables, or the balanced form's replicas of mid */
    size_t msplit_bytes;
    float *ys;
    unsigned *pub;
};

size_t moe_mid_ld(int inter) { return (size_t)((inter + 3) & ~3); }

/* bytes of one replica of the routed slots' mid tables in the balanced decode
 * form, 256-byte aligned */
size_t moe_copy_bytes(int topk, int inter) { return ((size_t)topk * mx_split_bytes(inter) + 255) & ~(size_t)255; }

/* Enqueue the decode MoE from device tables. */
/* Routed slots come from table[idx[k]] with weights w[k] (device arrays), or,
 * when `routed` is set, from the host arrays routed[k] / wv[k], passed by
 * value in the kernel arguments (MFMA path only). `ws` NULL: the library's
 * growing buffers (allocated here when too small). */
int enqueue_moe(const DSV4ExpertW *table, int n_experts, const int *idx,
                const float *w, int topk, const DSV4ExpertW *shared_dev,
                int shared_fmt, int shared_inter, int hidden, int inter,
                const float *x, float *out, float limit, hipStream_t st,
                const DSV4ExpertW *routed = nullptr, const float *wv = nullptr,
                const MoeWs *ws = nullptr)
{
    const size_t mid_ld = moe_mid_ld(inter);
    const bool mx = mx_expert_ok(FMT_FP4_E8M0, inter, hidden) && inter <= 2048 &&
                    topk <= MX_ROUTED_MAX && aligned16(x);
    if (routed && !mx)
        return fail("moe_decode_routed_dev: needs the MFMA path (FP4 experts, hidden and inter "
                    "multiples of 128, inter <= 2048, topk <= %d, x 16-byte aligned)", MX_ROUTED_MAX);
    const size_t sl = mx ? mx_split_bytes(inter) : 0;
    MoeWs m;
    if (ws) {
        m = *ws;
    } else {
        HIPCHK(g.mid.need(((size_t)topk * mid_ld + (shared_dev ? moe_mid_ld(shared_inter) : 0)) * 4),
               "mid alloc");
        if (shared_dev) HIPCHK(g.ys.need((size_t)hidden * 4), "shared output alloc");
        /* the split tables of the grid-ordered and two-launch forms, or the
         * balanced form's replicas of mid */
        if (mx)
            HIPCHK(g.msplit.need(std::max((size_t)topk * sl, BAL_MAX_COPIES * moe_copy_bytes(topk, inter))),
                   "mid split alloc");
        m.mid = (float *)g.mid.p;
        m.msplit = (uint8_t *)g.msplit.p;
        m.msplit_bytes = g.msplit.cap;
        m.ys = (float *)g.ys.p;
        m.pub = g.pub;
    }
    float *mid = m.mid;
    float *ys = nullptr;
    if (shared_dev) {
        ys = m.ys;
        float *smid = mid + (size_t)topk * mid_ld;
        if (enqueue_expert(*shared_dev, shared_fmt, shared_inter, hidden, x, smid,
                           ys, limit, st))
            return -1;
    }
    if (mx) {
        /* routed experts on the block-scaled MFMA: gate/up writes each slot's
         * mid split table, down reads it and combines in k order */
        GateUpMxArgs ga;
        memset(&ga, 0, sizeof ga);
        ga.table = table;
        ga.idx = idx;
        ga.n_experts = n_experts;
        ga.nslots = topk;
        ga.x = x;
        ga.mid = mid;
        ga.mid_ld = (int)mid_ld;
        ga.msplit = m.msplit;
        ga.msplit_ld = sl;
        ga.inter = inter;
        ga.hidden = hidden;
        ga.limit = limit;
        ga.status = g.st;
        if (routed) {
            ga.by_value = 1;
            for (int k = 0; k < topk; k++) ga.routed[k] = routed[k];
        }
        DownMxArgs da;
        memset(&da, 0, sizeof da);
        da.table = table;
        da.idx = idx;
        da.w = w;
        da.n_experts = n_experts;
        da.topk = topk;
        da.msplit = m.msplit;
        da.msplit_ld = sl;
        da.shared = ys;
        da.out = out;
        da.inter = inter;
        da.hidden = hidden;
        da.status = g.st;
        if (routed) {
            da.by_value = 1;
            for (int k = 0; k < topk; k++) {
                da.w2v[k] = routed[k].w2;
                da.wv[k] = wv[k];
            }
        }
        /* one launch: the down weight stream overlaps gate/up and there is
         * no second launch ramp. DSV4_HIP_DECODE_LAUNCHES selects the form
         * (same bits in all three): 0 the balanced one-launch form where it
         * applies, unset or 1 the grid-ordered one-launch form, 2 two
         * launches */
        const char *nl = getenv("DSV4_HIP_DECODE_LAUNCHES");
        const int form = nl ? atoi(nl) : 1;
        if (form != 2 && moe_one_ok(hidden, inter, topk)) {
            MoeOneArgs oa;
            memset(&oa, 0, sizeof oa);
            oa.gu = ga;
            oa.dn = da;
            oa.pub.count = m.pub;
            oa.pub.done = m.pub + ONE_COUNT_LINES * ONE_PUB_LINE_WORDS;
            oa.pub.leave = m.pub + (ONE_COUNT_LINES + 1) * ONE_PUB_LINE_WORDS;
            oa.midc = m.msplit;
            oa.copy_ld = moe_copy_bytes(topk, inter);
            oa.mid_copies = (int)std::min<size_t>(BAL_MAX_COPIES, m.msplit_bytes / moe_copy_bytes(topk, inter));
            /* DSV4_HIP_DECODE_SPIN: most polls of a down workgroup's wait
             * (default 2^20); 0 gives up without polling */
            const char *sp = getenv("DSV4_HIP_DECODE_SPIN");
            oa.spin_max = sp ? (unsigned)strtoul(sp, nullptr, 10) : 1u << 20;
            HIPCHK(moe_one_launch(oa, st, form == 0), "one-launch decode MoE");
            return 0;
        }
        HIPCHK(gateup_mx_launch(FMT_FP4_E8M0, ga, st), "routed gate/up launch");
        HIPCHK(down_mx_launch(da, st), "down/combine launch");
        return 0;
    }
    GateUpArgs ga;
    memset(&ga, 0, sizeof ga);
    ga.table = table;
    ga.idx = idx;
    ga.n_experts = n_experts;
    ga.nslots = topk;
    ga.x = x;
    ga.mid = mid;
    ga.mid_ld = (int)mid_ld;
    ga.inter = inter;
    ga.hidden = hidden;
    ga.limit = limit;
    ga.status = g.st;
    HIPCHK(gateup_launch(FMT_FP4_E8M0, ga, st), "routed gate/up launch");
    DownArgs da;
    memset(&da, 0, sizeof da);
    da.table = table;
    da.idx = idx;
    da.w = w;
    da.n_experts = n_experts;
    da.topk = topk;
    da.mid = mid;
    da.mid_ld = (int)mid_ld;
    da.shared = ys;
    da.out = out;
    da.inter = inter;
    da.hidden = hidden;
    da.status = g.st;
    HIPCHK(down_launch(da, st), "down/combine launch");
    return 0;
}

} // namespace

extern "C" {

int dsv4_hip_init(int device)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_init");
    const char *off = getenv("DSV4_HIP_DISABLE");
    if (off && *off && strcmp(off, "0") != 0)
        return fail("DSV4_HIP_DISABLE is set: the GPU backend is switched off");
    if (g.ready && g.device == device && !g.dead) return 0;
    if (g.ready) return fail("already initialised on device %d", g.device);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail("no HIP device");
    if (device < 0 || device >= n) return fail("device %d out of range (%d)", device, n);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail("hipGetDeviceProperties failed");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail("device %d is %s, this library is built for gfx950", device,
                    prop.gcnArchName);
    if (hipSetDevice(device) != hipSuccess) return fail("hipSetDevice failed");
    if (hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&g.side, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&g.side2, hipStreamNonBlocking) != hipSuccess)
        return fail("stream creation failed");
    if (hipEventCreateWithFlags(&g.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&g.join, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&g.fork2, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&g.join2, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&g.xq, hipEventDisableTiming) != hipSuccess)
        return fail("event creation failed");
    if (dev_malloc((void **)&g.status, 256) != hipSuccess) return fail("status alloc failed");
    if (hipMemset(g.status, 0, 256) != hipSuccess) return fail("status clear failed");
    if (dev_malloc((void **)&g.pub, ONE_PUB_BYTES) != hipSuccess) return fail("counter alloc failed");
    if (hipMemset(g.pub, 0, ONE_PUB_BYTES) != hipSuccess) return fail("counter clear failed");
    if (dev_malloc((void **)&g.rt_count, GATE_ROUTE_COUNTER_BYTES) != hipSuccess)
        return fail("counter alloc failed");
    if (hipMemset(g.rt_count, 0, GATE_ROUTE_COUNTER_BYTES) != hipSuccess)
        return fail("counter clear failed");
    g.st = g.status;
    /* this device's copy of the allocation-free entry point's scratch: its
     * address, looked up with the device current on every init, and its
     * hand-off words cleared (every launch leaves them at zero; an init after
     * a call that ended on a timeout starts from zero again) */
    if (device >= MAX_DEVICES) return fail("device %d beyond %d", device, MAX_DEVICES);
    {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail("scratch address lookup failed: %s", hipGetErrorString(e));
        if (hipMemset(p, 0, ONE_PUB_BYTES) != hipSuccess) return fail("scratch clear failed");
        if (hipDeviceSynchronize() != hipSuccess) return fail("scratch clear failed");
        scratch_ptr_of[device] = p;
    }

    g.device = device;
    g.ready = 1;
    g.dead = 0;
    return 0;
}

void dsv4_hip_shutdown(void)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (!g.ready) return;
    (void)hipDeviceSynchronize();
    for (auto &kv : g.regions) (void)hipFree(kv.second.dev);
    g.regions.clear();
    g.x.release(); g.y.release(); g.mid.release();
    g.table.release(); g.small.release(); g.ys.release(); g.gemm_ws.release();
    g.moe_ws.release(); g.x16.release(); g.msplit.release(); g.route.release();
    if (g.status) (void)hipFree(g.status);
    g.status = nullptr;
    if (g.pub) (void)hipFree(g.pub);
    g.pub = nullptr;
    if (g.rt_count) (void)hipFree(g.rt_count);
    g.rt_count = nullptr;
    if (g.stream) (void)hipStreamDestroy(g.stream);
    if (g.side) (void)hipStreamDestroy(g.side);
    if (g.side2) (void)hipStreamDestroy(g.side2);
    if (g.fork) (void)hipEventDestroy(g.fork);
    if (g.join) (void)hipEventDestroy(g.join);
    if (g.fork2) (void)hipEventDestroy(g.fork2);
    if (g.join2) (void)hipEventDestroy(g.join2);
    if (g.xq) (void)hipEventDestroy(g.xq);
    g.stream = g.side = g.side2 = nullptr;
    g.fork = g.join = g.fork2 = g.join2 = g.xq = nullptr;
    g.ready = 0;
    g.dead = 0;
    g.device = -1;
}

const char *dsv4_hip_last_error(void) { return g_err.c_str(); }

unsigned long long dsv4_hip_alloc_count(void) { return g_alloc_calls.load(std::memory_order_relaxed); }

int dsv4_hip_register(const void *host, size_t bytes)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (usable()) return -1;
    if (!host || !bytes) return fail("register: empty range");
    const uintptr_t a = (uintptr_t)host;
    auto it = g.regions.lower_bound(a);
    if (it != g.regions.end() && it->first < a + bytes)
        return fail("register: range overlaps a registered one");
    if (it != g.regions.begin()) {
        auto pv = std::prev(it);
        if (pv->first + pv->second.bytes > a)
            return fail("register: range overlaps a registered one");
    }
    void *dev = nullptr;
    hipError_t e = dev_malloc(&dev, bytes);
    if (e != hipSuccess) return fail("register: hipMalloc(%zu) failed", bytes);
    e = hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "register: upload");
    }
    g.regions[a] = Region{bytes, dev};
    return 0;
}

int dsv4_hip_unregister(const void *host)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (!g.ready) return fail("not initialised");
    auto it = g.regions.find((uintptr_t)host);
    if (it == g.regions.end()) return fail("unregister: unknown range");
    (void)hipStreamSynchronize(g.stream);
    (void)hipStreamSynchronize(g.side);
    (void)hipStreamSynchronize(g.side2);
    (void)hipFree(it->second.dev);
    g.regions.erase(it);
    return 0;
}

void *dsv4_hip_device_ptr(const void *p)
{
    std::lock_guard<std::mutex> lk(g.mu);
    return (void *)translate(p, 1);
}

/* y = W . x for nt tokens. BF16 matrices run the fp64-accumulating GEMV for
 * every nt. From MMQ_MFMA_MIN_TOKENS tokens on, packed matrices the grouped
 * kernel takes (rows, cols multiples of 128; FP8 with 128x128 blocks or FP4
 * with 1x32) run as one dense fp16-MFMA GEMM (x row-scaled by a power of two
 * and rounded to fp16, weights decoded exactly, fp32 accumulation): FP8 from
 * MMQ_SEAM_GEMM_MIN_TOKENS tokens on in the GEMM-shaped seam kernel (128 x
 * 256 tiles), else in the grouped kernel with one group (the same bits);
 * fewer tokens run the block-scaled MFMA GEMV where its geometry fits, else
 * the per-token VALU GEMV. The seam kernel's tiles fill the device only
 * from about 2048 tokens (4096 x 4096 FP8: 64 us from 128 to 1024 tokens,
 * 79 us at 2048), the grouped form's 64-token tiles from far fewer (32 us
 * at 128, 59 us at 1024, 82 us at 1536): the switch sits between. */
constexpr int MMQ_MFMA_MIN_TOKENS = 32;
constexpr int MMQ_SEAM_GEMM_MIN_TOKENS = 1280;
/* From this many tokens the block-scaled MFMA GEMV splits x once into its
 * e4m3 part tables (k_split_x_tab) and walks the token groups with each row
 * block's weights held (k_gemv_mx_tab), rather than every row block
 * splitting x and re-reading its weights per token group: 4096 x 4096 FP8,
 * 8 tokens 15.5 -> 12.3 us, 16 tokens 26.2 -> 16.7, 31 tokens 46.5 -> 24.1
 * (the same bits; at 2-4 tokens the extra launch costs what it saves). */
constexpr int MMQ_PRESPLIT_MIN_TOKENS = 5;

static int enqueue_mmq(const DSV4QMat &d, int fmt, const float *x, float *y, int nt, hipStream_t st)
{
    if (fmt >= FMT_GEN_FP8) {
        GemvGenArgs ga;
        ga.W = (const uint8_t *)d.w; ga.S = d.s; ga.x = x; ga.y = y;
        ga.rows = d.rows; ga.cols = d.cols; ga.blk_r = d.blk_r; ga.blk_c = d.blk_c; ga.nt = nt;
        HIPCHK(gemv_generic_launch(fmt, ga, st), "generic gemv launch");
        return 0;
    }
    if (fmt == FMT_BF16) {
        GemvBf16Args b;
        b.W = (const uint16_t *)d.w; b.x = x; b.y = y;
        b.rows = d.rows; b.cols = d.cols; b.nt = nt; b.x_ld = d.cols; b.y_ld = d.rows;
        HIPCHK(gemv_bf16_launch(b, st), "bf16 gemv launch");
        return 0;
    }
    const bool blocks = fmt == FMT_FP4_E8M0 ? d.blk_r == 1 : d.blk_r == 128;
    if (nt >= MMQ_MFMA_MIN_TOKENS && blocks && d.rows % 128 == 0 && d.cols % 128 == 0 &&
        ((uintptr_t)d.s & 3u) == 0) {
        const size_t xb = ((size_t)nt * d.cols * 2 + 255) & ~(size_t)255;
        HIPCHK(g.x16.need(xb + (size_t)nt * 4), "fp16 staging");
        uint16_t *x16 = (uint16_t *)g.x16.p;
        int *ex = (int *)((uint8_t *)g.x16.p + xb);
        HIPCHK(to_f16_rows_launch(x16, ex, x, nt, d.cols, st), "x fp16 launch");
        if (fmt != FMT_FP4_E8M0 && nt >= MMQ_SEAM_GEMM_MIN_TOKENS && aligned16(d.w) &&
            gemm_seam_ok(nt, d.rows, d.cols)) {
            SeamGemmArgs sg;
            sg.X = x16; sg.ex = ex; sg.W = (const uint8_t *)d.w; sg.Sw = d.s; sg.C = y;
            sg.M = nt; sg.N = d.rows; sg.K = d.cols;
            HIPCHK(gemm_seam_launch(sg, fmt == FMT_FP8_F32S, st), "seam GEMM launch");
            return 0;
        }
        GroupedArgs a;
        memset(&a, 0, sizeof a);
        a.m1 = d; a.nrows = nt; a.B = x16; a.bexp = ex; a.K = d.cols; a.N = d.rows; a.out = y;
        a.status = g.st;
        /* 16-token tiles give a small batch more workgroups (4096 x 4096
         * FP8: 23 us from 32 to 128 tokens, against 28-32 us in 64-token
         * tiles), 64-token tiles reuse each weight chunk more from about 200
         * tokens on (256 tokens: 33 against 37 us) */
        const int tt = nt <= 192 ? 1 : 4;
        const long tiles = (nt + grouped_rows_per_tile(tt) - 1) / grouped_rows_per_tile(tt);
        HIPCHK(grouped_launch(fmt, false, tt, a, tiles, st), "dense MFMA launch");
        return 0;
    }
    if (mx_gemv_ok(d, fmt, x)) {
        GemvMxArgs ga = gemv_mx_args(d, x, y, nt);
        if (nt >= MMQ_PRESPLIT_MIN_TOKENS) {
            HIPCHK(g.x16.need((size_t)nt * (d.cols / 128) * gemv_tab_chunk_bytes()), "split table");
            HIPCHK(split_x_tab_launch((uint8_t *)g.x16.p, x, d.cols, nt, d.cols, st), "x split launch");
            ga.tab = (const uint8_t *)g.x16.p;
        }
        HIPCHK(gemv_mx_launch(fmt, ga, st), "gemv launch");
        return 0;
    }
    HIPCHK(gemv_launch(fmt, gemv_args(d, x, y, nt), st), "gemv launch");
    return 0;
}

int dsv4_hip_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_mmq_n");
    if (usable()) return -1;
    if (nt <= 0) return 0;
    if (!x || !y) return fail("mmq_n: NULL x or y");
    DSV4QMat d;
    int fmt;
    if (resident(m, &d, "mmq_n", true, &fmt)) return -1;
    host_call();
    const size_t xb = (size_t)nt * m->cols * 4, yb = (size_t)nt * m->rows * 4;
    HIPCHK(g.x.need(xb), "x staging");
    HIPCHK(g.y.need(yb), "y staging");
    HIPCHK(hipMemcpyAsync(g.x.p, x, xb, hipMemcpyHostToDevice, g.stream), "x upload");
    if (enqueue_mmq(d, fmt, (const float *)g.x.p, (float *)g.y.p, nt, g.stream)) return -1;
    HIPCHK(hipMemcpyAsync(y, g.y.p, yb, hipMemcpyDeviceToHost, g.stream), "y download");
    return finish_host_call("mmq_n");
}

int dsv4_hip_mmq(float *y, const float *x, const DSV4QMat *m)
{
    return dsv4_hip_mmq_n(y, x, m, 1);
}

int dsv4_hip_mmq_n_dev(float *y, const float *x, const DSV4QMat *m, int nt,
                       void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_mmq_n_dev");
    if (usable()) return -1;
    if (nt <= 0) return 0;
    int fmt;
    if (check_qmat(m, "mmq_n_dev", &fmt, true)) return -1;
    if (!x || !y || !m->w || (fmt != FMT_BF16 && !m->s)) return fail("mmq_n_dev: NULL pointer");
    if (!aligned16(x) || !aligned16(m->w)) return fail("mmq_n_dev: x and W must be 16-byte aligned");
    dev_call();
    return enqueue_mmq(*m, fmt, x, y, nt, (hipStream_t)stream);
}

int dsv4_hip_mmq_multi_dev(const DSV4HipJob *jobs, int njobs, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_mmq_multi_dev");
    if (usable()) return -1;
    if (njobs < 0 || (njobs > 0 && !jobs)) return fail("mmq_multi_dev: %d jobs at %p", njobs, (const void *)jobs);
    std::vector<int> fmts((size_t)njobs, 0);
    for (int j = 0; j < njobs; j++) {
        const DSV4HipJob &jb = jobs[j];
        if (jb.n < 0) return fail("mmq_multi_dev: job %d has n = %d", j, jb.n);
        if (jb.n == 0) continue;
        if (check_qmat(jb.m, "mmq_multi_dev", &fmts[j], true)) return -1;
        if (!jb.x || !jb.y || !jb.m->w || (fmts[j] != FMT_BF16 && !jb.m->s))
            return fail("mmq_multi_dev: job %d has a NULL pointer", j);
        if (!aligned16(jb.x) || !aligned16(jb.m->w))
            return fail("mmq_multi_dev: job %d: x and W must be 16-byte aligned", j);
    }
    dev_call();
    const hipStream_t st = (hipStream_t)stream;
    /* one-token FP8 jobs that take the chunk-pair matvec, by format and launch
     * shape class, at most PX8_MAX_JOBS a launch; everything else one call
     * each */
    std::vector<GemvMxArgs> batch;
    std::vector<int> taken((size_t)njobs, 0);
    for (int j = 0; j < njobs; j++) {
        if (jobs[j].n == 0 || taken[j]) continue;
        const DSV4QMat &m = *jobs[j].m;
        /* the scale grid's width is only defined for the packed formats */
        const bool fp8 = fmts[j] == FMT_FP8_E8M0 || fmts[j] == FMT_FP8_F32S;
        const GemvMxArgs aj = fp8 ? gemv_mx_args(m, jobs[j].x, jobs[j].y, 1) : GemvMxArgs{};
        const bool pair = fp8 && jobs[j].n == 1 && mx_gemv_ok(m, fmts[j], jobs[j].x) && gemv_px8_ok(fmts[j], aj);
        if (!pair) {
            if (enqueue_mmq(m, fmts[j], jobs[j].x, jobs[j].y, jobs[j].n, st)) return -1;
            taken[j] = 1;
            continue;
        }
        batch.clear();
        for (int k = j; k < njobs && (int)batch.size() < PX8_MAX_JOBS; k++) {
            if (taken[k] || jobs[k].n != 1 || fmts[k] != fmts[j]) continue;   /* fmts[j] is FP8 */
            GemvMxArgs ak = gemv_mx_args(*jobs[k].m, jobs[k].x, jobs[k].y, 1);
            if (!mx_gemv_ok(*jobs[k].m, fmts[k], jobs[k].x) || !gemv_px8_ok(fmts[k], ak) ||
                gemv_px8_class(ak) != gemv_px8_class(aj))
                continue;
            batch.push_back(ak);
            taken[k] = 1;
        }
        HIPCHK(gemv_px8_multi_launch(fmts[j], batch.data(), (int)batch.size(), st), "multi-job matvec launch");
    }
    return 0;
}

int dsv4_hip_expert_forward(float *out, const float *x, const DSV4ExpertW *e,
                            int inter, float limit)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_expert_forward");
    if (usable()) return -1;
    if (!out || !x || !e) return fail("expert_forward: NULL pointer");
    int fmt, ei, eh;
    if (expert_geometry(e, &fmt, &ei, &eh, "expert_forward")) return -1;
    if (ei != inter) return fail("expert_forward: inter %d != w1 rows %d", inter, ei);
    DSV4ExpertW d;
    if (resident_expert(e, &d, "expert_forward")) return -1;
    host_call();
    HIPCHK(g.x.need((size_t)eh * 4), "x staging");
    HIPCHK(g.y.need((size_t)eh * 4), "y staging");
    HIPCHK(g.mid.need((size_t)inter * 4), "mid alloc");
    HIPCHK(hipMemcpyAsync(g.x.p, x, (size_t)eh * 4, hipMemcpyHostToDevice, g.stream), "x upload");
    if (enqueue_expert(d, fmt, inter, eh, (const float *)g.x.p, (float *)g.mid.p,
                       (float *)g.y.p, limit, g.stream))
        return -1;
    HIPCHK(hipMemcpyAsync(out, g.y.p, (size_t)eh * 4, hipMemcpyDeviceToHost, g.stream), "out download");
    return finish_host_call("expert_forward");
}

int dsv4_hip_moe_decode(float *out, const float *x, const DSV4ExpertW *const *ex,
                        const float *w, int topk, const DSV4ExpertW *shared,
                        float limit)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_decode");
    if (usable()) return -1;
    if (!out || !x || !ex || !w) return fail("moe_decode: NULL pointer");
    if (topk < 1 || topk > 16) return fail("moe_decode: topk %d outside 1..16", topk);
    DSV4ExpertW tab[16];
    int inter = 0, hidden = 0;
    for (int k = 0; k < topk; k++) {
        int fmt, ei, eh;
        if (!ex[k]) return fail("moe_decode: expert %d is NULL", k);
        if (expert_geometry(ex[k], &fmt, &ei, &eh, "moe_decode routed")) return -1;
        if (fmt != FMT_FP4_E8M0) return fail("moe_decode: routed experts must be FP4");
        if (k == 0) { inter = ei; hidden = eh; }
        else if (ei != inter || eh != hidden) return fail("moe_decode: routed shapes differ");
        if (inter / 2 > 2048) return fail("moe_decode: routed inter %d above 4096", inter);
        if (resident_expert(ex[k], &tab[k], "moe_decode routed")) return -1;
    }
    DSV4ExpertW sdev;
    int sfmt = -1, sinter = 0;
    if (shared) {
        int sh;
        if (expert_geometry(shared, &sfmt, &sinter, &sh, "moe_decode shared")) return -1;
        if (sh != hidden) return fail("moe_decode: shared hidden %d != %d", sh, hidden);
        if (resident_expert(shared, &sdev, "moe_decode shared")) return -1;
    }
    host_call();
    /* table, identity routing and weights in one small upload */
    const size_t tb = (size_t)topk * sizeof(DSV4ExpertW);
    const size_t ib = 16 * sizeof(int), wb = 16 * sizeof(float);
    HIPCHK(g.table.need(tb + ib + wb), "table alloc");
    unsigned char host[16 * sizeof(DSV4ExpertW) + 16 * 8];
    memcpy(host, tab, tb);
    int *hidx = (int *)(host + tb);
    float *hw = (float *)(host + tb + ib);
    for (int k = 0; k < topk; k++) { hidx[k] = k; hw[k] = w[k]; }
    HIPCHK(g.x.need((size_t)hidden * 4), "x staging");
    HIPCHK(g.y.need((size_t)hidden * 4), "y staging");
    HIPCHK(hipMemcpyAsync(g.table.p, host, tb + ib + wb, hipMemcpyHostToDevice, g.stream), "table upload");
    HIPCHK(hipMemcpyAsync(g.x.p, x, (size_t)hidden * 4, hipMemcpyHostToDevice, g.stream), "x upload");
    const unsigned char *tp = (const unsigned char *)g.table.p;
    if (enqueue_moe((const DSV4ExpertW *)tp, topk, (const int *)(tp + tb),
                    (const float *)(tp + tb + ib), topk, shared ? &sdev : nullptr,
                    sfmt, sinter, hidden, inter, (const float *)g.x.p,
                    (float *)g.y.p, limit, g.stream))
        return -1;
    HIPCHK(hipMemcpyAsync(out, g.y.p, (size_t)hidden * 4, hipMemcpyDeviceToHost, g.stream), "out download");
    return finish_host_call("moe_decode");
}

/* Checks of the device-routed decode MoE: geometry, topk and the shared
 * expert's format. */
static int decode_dev_checks(const char *what, const float *out, const float *x,
                      const DSV4ExpertW *experts, int n_experts, int topk,
                      const DSV4ExpertW *shared, int hidden, int inter, int *sfmt, int *sinter)
{
    if (!out || !x || !experts) return fail("%s: NULL pointer", what);
    if (topk < 1 || topk > 16) return fail("%s: topk %d outside 1..16", what, topk);
    if (n_experts < 1) return fail("%s: no experts", what);
    if (hidden % 32 || inter % 32 || hidden / 2 > 4096 || inter / 2 > 2048 || hidden <= 0 || inter <= 0)
        return fail("%s: unsupported hidden %d / inter %d", what, hidden, inter);
    if (!aligned16(x)) return fail("%s: x must be 16-byte aligned", what);
    *sfmt = -1;
    *sinter = 0;
    if (shared) {
        int sh;
        if (expert_geometry(shared, sfmt, sinter, &sh, what)) return -1;
        if (sh != hidden) return fail("%s: shared hidden %d != %d", what, sh, hidden);
        if (!aligned16(shared->w1.w) || !aligned16(shared->w3.w) || !aligned16(shared->w2.w))
            return fail("%s: shared weights must be 16-byte aligned", what);
    }
    return 0;
}

int dsv4_hip_moe_decode_dev(float *out, const float *x, const DSV4ExpertW *experts,
                            int n_experts, const int *idx, const float *w, int topk,
                            const DSV4ExpertW *shared, int hidden, int inter,
                            float limit, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_decode_dev");
    if (usable()) return -1;
    dev_call();
    if (!idx || !w) return fail("moe_decode_dev: NULL pointer");
    int sfmt, sinter;
    if (decode_dev_checks("moe_decode_dev", out, x, experts, n_experts, topk, shared, hidden,
                          inter, &sfmt, &sinter))
        return -1;
    return enqueue_moe(experts, n_experts, idx, w, topk, shared, sfmt, sinter,
                       hidden, inter, x, out, limit, (hipStream_t)stream);
}

/* Checks shared by the router entry points. */
static int route_checks(const char *what, int n_experts, int topk, const int64_t *tid2eid, int n_vocab)
{
    if (n_experts < 1 || n_experts > GATE_ROUTE_MAX_EXPERTS)
        return fail("%s: n_experts %d outside 1..%d", what, n_experts, GATE_ROUTE_MAX_EXPERTS);
    if (topk < 1 || topk > GATE_ROUTE_MAX_TOPK || topk > n_experts)
        return fail("%s: topk %d outside 1..%d", what, topk,
                    std::min(GATE_ROUTE_MAX_TOPK, n_experts));
    if (tid2eid && n_vocab < 1) return fail("%s: hash routing needs n_vocab >= 1", what);
    return 0;
}

int dsv4_hip_route_dev(int *idx, float *w, float *orig, const float *scores, int n,
                       const float *bias, const int64_t *tid2eid, int n_vocab,
                       const int *token_ids, int n_experts, int topk, float route_scale,
                       void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_route_dev");
    if (usable()) return -1;
    dev_call();
    if (n < 0) return fail("route_dev: n %d < 0", n);
    if (n == 0) return 0;
    if (!idx || !w || !scores) return fail("route_dev: NULL pointer");
    if (route_checks("route_dev", n_experts, topk, tid2eid, n_vocab)) return -1;
    if (tid2eid && !token_ids) return fail("route_dev: hash routing needs token_ids");
    GateRouteArgs a;
    memset(&a, 0, sizeof a);
    a.scores = scores;
    a.scores_ld = n_experts;
    a.n = n;
    a.bias = bias;
    a.tid2eid = tid2eid;
    a.n_vocab = n_vocab;
    a.token_ids = token_ids;
    a.n_experts = n_experts;
    a.topk = topk;
    a.route_scale = route_scale;
    a.idx = idx;
    a.w = w;
    a.orig = orig;
    a.status = g.st;
    HIPCHK(gate_route_launch(a, (hipStream_t)stream), "route launch");
    return 0;
}

int dsv4_hip_moe_layer_dev(float *out, const float *x, const DSV4QMat *gate,
                           const float *bias, const int64_t *tid2eid, int n_vocab, int token_id,
                           float route_scale, const DSV4ExpertW *experts, int n_experts, int topk,
                           const DSV4ExpertW *shared, int hidden, int inter, float limit,
                           int *idx_out, float *w_out, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_layer_dev");
    if (usable()) return -1;
    dev_call();
    int gfmt, sfmt, sinter;
    if (check_qmat(gate, "moe_layer_dev gate", &gfmt)) return -1;
    if (!gate->w || (gfmt != FMT_BF16 && !gate->s)) return fail("moe_layer_dev: NULL gate pointer");
    if (gate->rows != n_experts || gate->cols != hidden)
        return fail("moe_layer_dev: gate is [%d x %d], expected [%d x %d]", gate->rows,
                    gate->cols, n_experts, hidden);
    if (!aligned16(gate->w)) return fail("moe_layer_dev: gate weights must be 16-byte aligned");
    if (route_checks("moe_layer_dev", n_experts, topk, tid2eid, n_vocab)) return -1;
    if (decode_dev_checks("moe_layer_dev", out, x, experts, n_experts, topk, shared, hidden,
                          inter, &sfmt, &sinter))
        return -1;
    const hipStream_t st = (hipStream_t)stream;
    const size_t sb = ((size_t)n_experts * 4 + 255) & ~(size_t)255;
    HIPCHK(g.route.need(3 * sb + 2 * 256), "router workspace");
    float *scores = (float *)g.route.p;
    int *idx = idx_out ? idx_out : (int *)((uint8_t *)g.route.p + 3 * sb);
    float *w = w_out ? w_out : (float *)((uint8_t *)g.route.p + 3 * sb + 256);
    /* a BF16 gate of up to 4096 columns runs fused with the router (one
     * launch); any other gate runs through dsv4_mmq's kernels first */
    const bool fused = gfmt == FMT_BF16 && hidden <= 4096;
    if (!fused && enqueue_mmq(*gate, gfmt, x, scores, 1, st)) return -1;
    GateRouteArgs a;
    memset(&a, 0, sizeof a);
    if (fused) {
        a.gate_w = (const uint16_t *)gate->w;
        a.x = x;
        a.cols = hidden;
        a.ws_orig = (float *)((uint8_t *)g.route.p + sb);
        a.ws_biased = (float *)((uint8_t *)g.route.p + 2 * sb);
        a.counter = g.rt_count;
    }
    a.scores = scores;
    a.scores_ld = n_experts;
    a.n = 1;
    a.bias = bias;
    a.tid2eid = tid2eid;
    a.n_vocab = n_vocab;
    a.token_id = token_id;
    a.n_experts = n_experts;
    a.topk = topk;
    a.route_scale = route_scale;
    a.idx = idx;
    a.w = w;
    a.status = g.st;
    HIPCHK(gate_route_launch(a, st), "route launch");
    /* everything on the caller's stream: a fork of the shared expert onto a
     * second stream cost about 10 us per event wait, more than it hid */
    return enqueue_moe(experts, n_experts, idx, w, topk, shared, sfmt, sinter,
                       hidden, inter, x, out, limit, st);
}

/* Checks of the host-routed decode entry points: the topk descriptors and
 * weights picked by the host routing ids, and the shared expert's format. */
static int routed_checks(const char *what, const float *out, const float *x, const DSV4ExpertW *experts,
                  int n_experts, const int *idx, const float *w, int topk,
                  const DSV4ExpertW *shared, int hidden, int inter, DSV4ExpertW *routed,
                  float *wv, int *sfmt, int *sinter)
{
    if (!out || !x || !experts || !idx || !w) return fail("%s: NULL pointer", what);
    if (topk < 1 || topk > MX_ROUTED_MAX)
        return fail("%s: topk %d outside 1..%d", what, topk, MX_ROUTED_MAX);
    if (n_experts < 1) return fail("%s: no experts", what);
    if (!aligned16(x)) return fail("%s: x must be 16-byte aligned", what);
    for (int k = 0; k < topk; k++) {
        const int id = idx[k];
        if (id < 0 || id >= n_experts)
            return fail("%s: routing id %d of slot %d outside 0..%d", what, id, k, n_experts - 1);
        int f, ei, eh;
        if (expert_geometry(&experts[id], &f, &ei, &eh, what)) return -1;
        if (f != FMT_FP4_E8M0 || ei != inter || eh != hidden)
            return fail("%s: expert %d is not FP4 [%d x %d]", what, id, inter, hidden);
        routed[k] = experts[id];
        wv[k] = w[k];
    }
    *sfmt = -1;
    *sinter = 0;
    if (shared) {
        int sh;
        if (expert_geometry(shared, sfmt, sinter, &sh, what)) return -1;
        if (sh != hidden) return fail("%s: shared hidden %d != %d", what, sh, hidden);
        if (!aligned16(shared->w1.w) || !aligned16(shared->w3.w) || !aligned16(shared->w2.w))
            return fail("%s: shared weights must be 16-byte aligned", what);
    }
    return 0;
}

int dsv4_hip_moe_decode_routed_dev(float *out, const float *x, const DSV4ExpertW *experts,
                                   int n_experts, const int *idx, const float *w, int topk,
                                   const DSV4ExpertW *shared, int hidden, int inter,
                                   float limit, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_decode_routed_dev");
    if (usable()) return -1;
    dev_call();
    DSV4ExpertW routed[MX_ROUTED_MAX];
    float wv[MX_ROUTED_MAX];
    int sfmt, sinter;
    if (routed_checks("moe_decode_routed_dev", out, x, experts, n_experts, idx, w, topk, shared,
                      hidden, inter, routed, wv, &sfmt, &sinter))
        return -1;
    return enqueue_moe(nullptr, n_experts, nullptr, nullptr, topk, shared, sfmt, sinter, hidden,
                       inter, x, out, limit, (hipStream_t)stream, routed, wv);
}

int dsv4_hip_moe_decode_routed_noalloc_dev(float *out, const float *x, const DSV4ExpertW *experts,
                                           int n_experts, const int *idx, const float *w, int topk,
                                           const DSV4ExpertW *shared, int hidden, int inter,
                                           float limit, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_decode_routed_noalloc_dev");
    if (usable()) return -1;
    dev_call();
    const char *what = "moe_decode_routed_noalloc_dev";
    uint8_t *base = (uint8_t *)scratch_ptr_of[g.device];
    if (!base) return fail("%s: the device scratch is not mapped", what);
    DSV4ExpertW routed[MX_ROUTED_MAX];
    float wv[MX_ROUTED_MAX];
    int sfmt, sinter;
    if (routed_checks(what, out, x, experts, n_experts, idx, w, topk, shared, hidden, inter, routed,
                      wv, &sfmt, &sinter))
        return -1;
    if (inter <= 0 || inter % 128 || inter > 2048 || hidden <= 0 || hidden % 128 || hidden > 4096 ||
        (shared && sinter > 2048))
        return fail("%s: the device scratch holds inter <= 2048 and hidden <= 4096 in multiples "
                    "of 128 (shared inter <= 2048); got inter %d, hidden %d, shared inter %d",
                    what, inter, hidden, sinter);
    /* layout: hand-off words, mid rows (routed then shared), split tables,
     * shared output; each part 256-byte aligned */
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t o_mid = up(ONE_PUB_BYTES);
    const size_t o_split = o_mid + up(((size_t)topk * moe_mid_ld(inter) +
                                       (shared ? moe_mid_ld(sinter) : 0)) * 4);
    const size_t o_ys = o_split + up((size_t)topk * mx_split_bytes(inter));
    const size_t need = o_ys + (shared ? (size_t)hidden * 4 : 0);
    if (need > SCRATCH_BYTES)
        return fail("%s: needs %zu bytes of device scratch, the maximum is %zu", what, need,
                    (size_t)SCRATCH_BYTES);
    MoeWs ws;
    ws.pub = (unsigned *)base;
    ws.mid = (float *)(base + o_mid);
    ws.msplit = base + o_split;
    ws.msplit_bytes = o_ys - o_split;
    ws.ys = (float *)(base + o_ys);
    return enqueue_moe(nullptr, n_experts, nullptr, nullptr, topk, shared, sfmt, sinter, hidden,
                       inter, x, out, limit, (hipStream_t)stream, routed, wv, &ws);
}

/* ------------------------------------------- checkpoint experts --- */

/* experts.idx record (tools/pack_trunk.py writes "<iiqq"). */
struct ExpLoc {
    int32_t shard, pad;
    int64_t off, nbytes;
};
static_assert(sizeof(ExpLoc) == 24, "experts.idx record");
constexpr int EXP_TENSORS = 6;                 /* w1, w1 scales, w2, w2 scales, w3, w3 scales */

/* The *.safetensors files of dir in strcmp order: shard i of the index. */
static int list_shards(const char *dir, std::vector<std::string> &out)
{
    DIR *d = opendir(dir);
    if (!d) return fail("load_experts: cannot open directory %s", dir);
    while (struct dirent *e = readdir(d)) {
        const size_t n = strlen(e->d_name);
        if (n >= 12 && strcmp(e->d_name + n - 12, ".safetensors") == 0)
            out.push_back(std::string(dir) + "/" + e->d_name);
    }
    closedir(d);
    if (out.empty()) return fail("load_experts: no .safetensors files in %s", dir);
    std::sort(out.begin(), out.end(), [](const std::string &a, const std::string &b) {
        return strcmp(a.c_str(), b.c_str()) < 0;
    });
    return 0;
}

/* The layer's records: n_experts x 6, in the packer's tensor order. */
static int read_expert_index(const char *index_dir, int layer, std::vector<ExpLoc> &loc, int *n_experts)
{
    const std::string path = std::string(index_dir) + "/experts.idx";
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return fail("load_experts: cannot open %s", path.c_str());
    char magic[8];
    int32_t nl = 0, ne = 0;
    int rc = 0;
    if (fread(magic, 1, 8, f) != 8 || memcmp(magic, "DSV4EXP1", 8) != 0)
        rc = fail("load_experts: %s is not an experts index (magic DSV4EXP1)", path.c_str());
    else if (fread(&nl, 4, 1, f) != 1 || fread(&ne, 4, 1, f) != 1 || nl <= 0 || ne <= 0)
        rc = fail("load_experts: %s has a bad header", path.c_str());
    else if (layer < 0 || layer >= nl)
        rc = fail("load_experts: layer %d outside 0..%d", layer, nl - 1);
    if (!rc) {
        const long rec = (long)ne * EXP_TENSORS;
        loc.resize((size_t)rec);
        if (fseek(f, 16 + (long)layer * rec * (long)sizeof(ExpLoc), SEEK_SET) != 0 ||
            fread(loc.data(), sizeof(ExpLoc), (size_t)rec, f) != (size_t)rec)
            rc = fail("load_experts: %s is short for layer %d", path.c_str(), layer);
        *n_experts = ne;
    }
    fclose(f);
    return rc;
}

/* Device arenas handed out by dsv4_hip_load_experts. */
static std::map<uintptr_t, size_t> g_expert_arenas;

/* Shared checks of the FP8 GEMM entry points; returns the weight format. */
static int gemm_checks(const void *C, const void *A, int M, const DSV4QMat *W, const char *what, int *fmt)
{
    if (!C || !A || !W || !W->w || !W->s) return fail("%s: NULL pointer", what);
    *fmt = qmat_fmt(W);
    if ((*fmt != FMT_FP8_E8M0 && *fmt != FMT_FP8_F32S) || W->blk_r != 128 || W->blk_c != 128)
        return fail("%s: W must be e4m3 with 128x128 block scales", what);
    if (M <= 0 || W->cols % 128 || W->rows % 128)
        return fail("%s: need M > 0 and rows, cols multiples of 128 (got M %d, %d x %d)", what,
                    M, W->rows, W->cols);
    if (!aligned16(A) || !aligned16(W->w) || ((uintptr_t)C & 15u))
        return fail("%s: A, C and W must be 16-byte aligned", what);
    return 0;
}

/* Sa holds one fp32 per (token, 128-wide K block), block-major [K/128][M]. */
static int enqueue_gemm(void *C, int out_bf16, const uint8_t *Aq, const float *Sa, int M,
                 const DSV4QMat *W, int fmt, hipStream_t st)
{
    GemmArgs ga;
    ga.Aq = Aq; ga.Sa = Sa; ga.W = (const uint8_t *)W->w; ga.Sw = W->s; ga.C = C;
    ga.M = M; ga.N = W->rows; ga.K = W->cols; ga.ldc = W->rows;
    ga.sa_tok = 1;
    ga.sa_kb = M;
    HIPCHK(gemm_fp8_launch(ga, fmt == FMT_FP8_F32S, out_bf16 != 0, st), "gemm launch");
    return 0;
}

int dsv4_hip_gemm_fp8_dev(void *C, int out_bf16, const void *A, int a_bf16, int M,
                          const DSV4QMat *W, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_gemm_fp8_dev");
    if (usable()) return -1;
    dev_call();
    int fmt;
    if (gemm_checks(C, A, M, W, "gemm_fp8_dev", &fmt)) return -1;
    const int K = W->cols;
    const size_t qbytes = ((size_t)M * K + 255) & ~(size_t)255;
    HIPCHK(g.gemm_ws.need(qbytes + (size_t)M * (K / 128) * 4), "gemm workspace");
    uint8_t *Aq = (uint8_t *)g.gemm_ws.p;
    float *Sa = (float *)(Aq + qbytes);
    hipStream_t st = (hipStream_t)stream;
    HIPCHK(quant_act_fp8_1x128_launch(Aq, Sa, A, M, K, a_bf16 != 0, true, st),
           "activation quant launch");
    return enqueue_gemm(C, out_bf16, Aq, Sa, M, W, fmt, st);
}

int dsv4_hip_gemm_fp8q_dev(void *C, int out_bf16, const uint8_t *Aq, const float *Sa,
                           int M, const DSV4QMat *W, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_gemm_fp8q_dev");
    if (usable()) return -1;
    dev_call();
    int fmt;
    if (gemm_checks(C, Aq, M, W, "gemm_fp8q_dev", &fmt)) return -1;
    if (!Sa) return fail("gemm_fp8q_dev: NULL scales");
    return enqueue_gemm(C, out_bf16, Aq, Sa, M, W, fmt, (hipStream_t)stream);
}

/* The hardware-scaled GEMM: W must carry E8M0 128 x 128 block scales. As
 * token-major [M][K / 32] bytes, or block-major (s_blk_major: one dword per
 * token and 128-wide K block, [K / 128][M] dwords). */
static int enqueue_gemm_mx(void *C, int out_bf16, const uint8_t *Aq, const uint8_t *As, int M,
                    const DSV4QMat *W, bool s_blk_major, hipStream_t st)
{
    GemmArgs ga;
    ga.Aq = Aq; ga.Sa = (const float *)As; ga.W = (const uint8_t *)W->w; ga.Sw = W->s; ga.C = C;
    ga.M = M; ga.N = W->rows; ga.K = W->cols; ga.ldc = W->rows;
    ga.sa_tok = s_blk_major ? 1 : W->cols / 128;
    ga.sa_kb = s_blk_major ? M : 1;
    HIPCHK(gemm_mx_launch(ga, out_bf16 != 0, st), "gemm launch");
    return 0;
}

void *dsv4_hip_load_experts(const char *model_dir, const char *index_dir, int layer, int hidden,
                            int inter, DSV4ExpertW *table, int max_experts, int *n_experts)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_load_experts");
    if (!model_dir || !index_dir || !table || !n_experts) {
        fail("load_experts: NULL argument");
        return nullptr;
    }
    if (hidden <= 0 || inter <= 0 || hidden % 32 || inter % 32) {
        fail("load_experts: hidden %d and inter %d must be positive multiples of 32", hidden, inter);
        return nullptr;
    }
    /* the index and the shard list first: a bad checkpoint fails before
     * any device memory is touched */
    std::vector<ExpLoc> loc;
    int ne = 0;
    if (read_expert_index(index_dir, layer, loc, &ne)) return nullptr;
    if (ne > max_experts) {
        fail("load_experts: the index has %d experts, the table holds %d", ne, max_experts);
        return nullptr;
    }
    std::vector<std::string> shards;
    if (list_shards(model_dir, shards)) return nullptr;
    /* one slot per expert as the reference's cache lays it out
     * (src/60_cache/dsv4_cache_geom.c:14-31): scales s1 s2 s3, then weights
     * w1 w2 w3; slots 4096-byte aligned */
    const int64_t H = hidden, I = inter;
    const int64_t wb[3] = {I * (H / 2), H * (I / 2), I * (H / 2)};
    const int64_t sb[3] = {I * (H / 32), H * (I / 32), I * (H / 32)};
    int64_t off_s[3], off_w[3], at = 0;
    for (int i = 0; i < 3; i++) { off_s[i] = at; at += sb[i]; }
    for (int i = 0; i < 3; i++) { off_w[i] = at; at += wb[i]; }
    const size_t slot = (size_t)((at + 4095) / 4096 * 4096);
    /* index order w1 w1s w2 w2s w3 w3s -> (matrix, is scale) */
    const int mat_of[EXP_TENSORS] = {0, 0, 1, 1, 2, 2};
    for (int e = 0; e < ne; e++)
        for (int j = 0; j < EXP_TENSORS; j++) {
            const ExpLoc &l = loc[(size_t)e * EXP_TENSORS + j];
            const int64_t want = (j & 1) ? sb[mat_of[j]] : wb[mat_of[j]];
            if (l.shard < 0 || l.shard >= (int)shards.size() || l.off < 0 || l.nbytes != want) {
                fail("load_experts: layer %d expert %d tensor %d: shard %d, %lld bytes (want %lld, %zu shards)",
                     layer, e, j, l.shard, (long long)l.nbytes, (long long)want, shards.size());
                return nullptr;
            }
        }
    if (usable()) return nullptr;
    std::vector<int> fds(shards.size(), -1);
    auto close_all = [&]() { for (int fd : fds) if (fd >= 0) close(fd); };
    for (size_t i = 0; i < shards.size(); i++) {
        fds[i] = open(shards[i].c_str(), O_RDONLY);
        if (fds[i] < 0) {
            close_all();
            fail("load_experts: cannot open %s", shards[i].c_str());
            return nullptr;
        }
    }
    uint8_t *arena = nullptr, *stage = nullptr;
    if (dev_malloc((void **)&arena, slot * (size_t)ne) != hipSuccess ||
        hipHostMalloc((void **)&stage, slot, hipHostMallocDefault) != hipSuccess) {
        if (arena) (void)hipFree(arena);
        close_all();
        fail("load_experts: cannot allocate %zu bytes of device arena", slot * (size_t)ne);
        return nullptr;
    }
    bool ok = true;
    for (int e = 0; e < ne && ok; e++) {
        for (int j = 0; j < EXP_TENSORS && ok; j++) {
            const ExpLoc &l = loc[(size_t)e * EXP_TENSORS + j];
            uint8_t *dst = stage + ((j & 1) ? off_s[mat_of[j]] : off_w[mat_of[j]]);
            int64_t done = 0;
            while (done < l.nbytes) {
                const ssize_t r = pread(fds[(size_t)l.shard], dst + done, (size_t)(l.nbytes - done),
                                        (off_t)(l.off + done));
                if (r <= 0) {
                    ok = false;
                    fail("load_experts: short read of layer %d expert %d tensor %d from %s", layer, e, j,
                         shards[(size_t)l.shard].c_str());
                    break;
                }
                done += r;
            }
        }
        if (ok && hipMemcpy(arena + (size_t)e * slot, stage, (size_t)at, hipMemcpyHostToDevice) != hipSuccess) {
            ok = false;
            fail("load_experts: upload of expert %d failed", e);
        }
    }
    close_all();
    (void)hipHostFree(stage);
    if (!ok) {
        (void)hipFree(arena);
        return nullptr;
    }
    const int64_t rows[3] = {I, H, I}, cols[3] = {H, I, H};
    for (int e = 0; e < ne; e++) {
        uint8_t *b = arena + (size_t)e * slot;
        DSV4QMat *m[3] = {&table[e].w1, &table[e].w2, &table[e].w3};
        for (int i = 0; i < 3; i++) {
            memset(m[i], 0, sizeof *m[i]);
            m[i]->wdt = DSV4_WFP4;
            m[i]->rows = (int)rows[i];
            m[i]->cols = (int)cols[i];
            m[i]->blk_r = 1;
            m[i]->blk_c = 32;
            m[i]->w = b + off_w[i];
            m[i]->s = b + off_s[i];
        }
    }
    g_expert_arenas[(uintptr_t)arena] = slot * (size_t)ne;
    *n_experts = ne;
    return arena;
}

int dsv4_hip_free_experts(void *arena)
{
    std::lock_guard<std::mutex> lk(g.mu);
    auto it = g_expert_arenas.find((uintptr_t)arena);
    if (it == g_expert_arenas.end()) return fail("free_experts: not an arena of dsv4_hip_load_experts");
    (void)hipDeviceSynchronize();
    (void)hipFree(arena);
    g_expert_arenas.erase(it);
    return 0;
}

int dsv4_hip_gemm_mxfp8_dev(void *C, int out_bf16, const void *A, int a_bf16, int M,
                            const DSV4QMat *W, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_gemm_mxfp8_dev");
    if (usable()) return -1;
    dev_call();
    int fmt;
    if (gemm_checks(C, A, M, W, "gemm_mxfp8_dev", &fmt)) return -1;
    if (fmt != FMT_FP8_E8M0) return fail("gemm_mxfp8_dev: W must carry E8M0 block scales (DSV4_WFP8)");
    const int K = W->cols;
    const size_t qbytes = ((size_t)M * K + 255) & ~(size_t)255;
    HIPCHK(g.gemm_ws.need(qbytes + (size_t)M * (K / 32)), "gemm workspace");
    uint8_t *Aq = (uint8_t *)g.gemm_ws.p;
    uint8_t *As = Aq + qbytes;
    hipStream_t st = (hipStream_t)stream;
    HIPCHK(quant_act_mxfp8_launch(Aq, As, A, M, K, st, a_bf16 != 0, true), "activation quant launch");
    return enqueue_gemm_mx(C, out_bf16, Aq, As, M, W, true, st);
}

int dsv4_hip_gemm_mxfp8q_dev(void *C, int out_bf16, const uint8_t *Aq, const uint8_t *As,
                             int M, const DSV4QMat *W, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_gemm_mxfp8q_dev");
    if (usable()) return -1;
    dev_call();
    int fmt;
    if (gemm_checks(C, Aq, M, W, "gemm_mxfp8q_dev", &fmt)) return -1;
    if (fmt != FMT_FP8_E8M0) return fail("gemm_mxfp8q_dev: W must carry E8M0 block scales (DSV4_WFP8)");
    if (!As) return fail("gemm_mxfp8q_dev: NULL scales");
    return enqueue_gemm_mx(C, out_bf16, Aq, As, M, W, false, (hipStream_t)stream);
}

/* ------------------------------------------------------ grouped MoE --- */

/* 16-row tiles when buckets are small (batched decode: few tokens per expert,
 * weight streaming dominates and occupancy matters), 128-row tiles otherwise
 * (prefill: weights are reused across a tile's rows). */
static int grouped_tt(long pairs) { return pairs <= 4096 ? 1 : 8; }

static int enqueue_moe_grouped(float *out, const float *x, int n, const DSV4ExpertW *table,
                        int n_experts, const int *idx, const float *w, int topk,
                        const DSV4ExpertW *shared, int sfmt, int sinter, int hidden,
                        int inter, float limit, hipStream_t st)
{
    const long P = (long)n * topk;
    int tt = grouped_tt(P);
    /* the 128-row kernel takes 256 down rows per workgroup and 31-bit offsets */
    if (tt == 8 && (hidden % 256 || (size_t)P * inter * 2 >= (1u << 31) ||
                    (size_t)n * hidden * 2 >= (1u << 31) || (size_t)inter * hidden / 2 >= (1u << 31)))
        tt = 4;
    const int trows = grouped_rows_per_tile(tt);
    size_t off = 0;
    auto take = [&](size_t b) { const size_t o = off; off += (b + 255) & ~(size_t)255; return o; };
    /* every bucket adds at most one partial tile */
    const long max_tiles = (P + trows - 1) / trows + n_experts;
    const size_t o_grp = take((size_t)(n_experts + 1) * 4), o_tp = take((size_t)(n_experts + 1) * 4);
    const size_t o_tg = take((size_t)(max_tiles + 4) * sizeof(TileRec));
    const size_t o_pos = take((size_t)P * 4), o_row = take((size_t)P * 4);
    const size_t o_ch = take(route_chist_bytes(P, n_experts));
    const size_t o_x16 = take((size_t)n * hidden * 2), o_mid = take((size_t)P * inter * 2);
    const size_t o_y = take((size_t)P * hidden * 4), o_ex = take((size_t)n * 4);
    size_t o_smid = 0, o_ys = 0;
    if (shared) {
        o_smid = take((size_t)n * sinter * 2);
        o_ys = take((size_t)n * hidden * 4);
    }
    HIPCHK(g.moe_ws.need(off), "grouped MoE workspace");
    uint8_t *ws = (uint8_t *)g.moe_ws.p;
    int *grp = (int *)(ws + o_grp), *tp = (int *)(ws + o_tp);
    TileRec *tg = (TileRec *)(ws + o_tg);
    int *pos = (int *)(ws + o_pos), *row = (int *)(ws + o_row);
    uint16_t *x16 = (uint16_t *)(ws + o_x16), *mid = (uint16_t *)(ws + o_mid);
    float *y = (float *)(ws + o_y);
    int *ex = (int *)(ws + o_ex);

    RouteArgs ra;
    ra.idx = idx; ra.npairs = (int)P; ra.topk = topk; ra.n_experts = n_experts;
    ra.tile_rows = trows; ra.grp_off = grp; ra.tile_pre = tp; ra.tile_rec = tg; ra.pos = pos;
    ra.row_tok = row;
    ra.row_k = nullptr;
    ra.chist = (int *)(ws + o_ch);
    ra.status = g.st;
    /* A large x goes to fp16 on the side stream, beside the routing
     * permutation on this one (neither reads the other's output), and this
     * stream waits for it before the routed launches. A small one converts
     * here first: the conversion then takes less than that cross-stream wait
     * (about 10 us between kernels). Either way the shared expert, which
     * needs only x16, runs on the side stream after it, overlaps the routed
     * launches and is joined before the combine. */
    const bool fork_x = (size_t)n * hidden > ((size_t)1 << 22);
    if (!fork_x) HIPCHK(to_f16_rows_launch(x16, ex, x, n, hidden, st), "x fp16 launch");
    HIPCHK(hipEventRecord(g.fork, st), "fork record");
    HIPCHK(hipStreamWaitEvent(g.side, g.fork, 0), "fork wait");
    if (fork_x) {
        HIPCHK(to_f16_rows_launch(x16, ex, x, n, hidden, g.side), "x fp16 launch");
        HIPCHK(hipEventRecord(g.xq, g.side), "convert record");
    }
    HIPCHK(moe_route_launch(ra, st), "route launch");
    if (fork_x) HIPCHK(hipStreamWaitEvent(st, g.xq, 0), "convert wait");

    float *ys = nullptr;
    if (shared) {
        uint16_t *smid = (uint16_t *)(ws + o_smid);
        ys = (float *)(ws + o_ys);
        const int stt = n <= 64 ? 1 : 4;     /* enough workgroups for a small batch */
        const long stiles = (n + grouped_rows_per_tile(stt) - 1) / grouped_rows_per_tile(stt);
        GroupedArgs sa;
        memset(&sa, 0, sizeof sa);
        sa.m1 = shared->w1; sa.m3 = shared->w3; sa.nrows = n; sa.B = x16; sa.bexp = ex;
        sa.K = hidden; sa.N = sinter; sa.out = smid; sa.limit = limit; sa.status = g.st;
        HIPCHK(grouped_launch(sfmt, true, stt, sa, stiles, g.side), "shared gate/up launch");
        sa.m1 = shared->w2; sa.B = smid; sa.bexp = nullptr; sa.K = sinter; sa.N = hidden; sa.out = ys;
        HIPCHK(grouped_launch(sfmt, false, stt, sa, stiles, g.side), "shared down launch");
        HIPCHK(hipEventRecord(g.join, g.side), "join record");
    }

    GroupedArgs ga;
    memset(&ga, 0, sizeof ga);
    ga.table = table; ga.n_experts = n_experts; ga.grp_off = grp; ga.tile_pre = tp; ga.tile_rec = tg;
    ga.row_tok = row; ga.nrows = n; ga.B = x16; ga.bexp = ex; ga.K = hidden; ga.N = inter;
    ga.out = mid; ga.limit = limit; ga.status = g.st;
    HIPCHK(grouped_launch(FMT_FP4_E8M0, true, tt, ga, max_tiles, st), "routed gate/up launch");
    ga.row_tok = nullptr; ga.bexp = nullptr;
    ga.nrows = (int)P; ga.B = mid; ga.K = inter; ga.N = hidden; ga.out = y;
    HIPCHK(grouped_launch(FMT_FP4_E8M0, false, tt, ga, max_tiles, st), "routed down launch");

    if (shared) HIPCHK(hipStreamWaitEvent(st, g.join, 0), "join wait");
    CombineArgs ca;
    ca.out = out; ca.Y = y; ca.YS = ys; ca.w = w; ca.pos = pos;
    ca.n = n; ca.topk = topk; ca.hidden = hidden;
    HIPCHK(moe_combine_launch(ca, st), "combine launch");
    return 0;
}

/* An FP8 shared expert over n tokens as the reference's GPU prefill runs it
 * (src/80_prefill/dsv4_prefill_moe.c:40-58): x quantized 1x128 to e4m3 (xq,
 * xs), the w1 and w3 GEMMs into fp32 gate and up, SwiGLU with mid's 1x128
 * quantization in one pass (mq, ms block-major), and the w2 GEMM into ys;
 * ys == NULL stops after mid. */
static int enqueue_shared_fp8q(float *ys, uint8_t *mq, float *ms, const float *x, int n, const DSV4ExpertW *sh,
                        int sfmt, int sinter, int hidden, float limit, uint8_t *xq, float *xs, float *gate,
                        float *up, hipStream_t st)
{
    HIPCHK(quant_act_fp8_1x128_launch(xq, xs, x, n, hidden, false, true, st), "shared x FP8 launch");
    if (enqueue_gemm(gate, 0, xq, xs, n, &sh->w1, sfmt, st) || enqueue_gemm(up, 0, xq, xs, n, &sh->w3, sfmt, st))
        return -1;
    HIPCHK(swiglu_quant_fp8_launch(mq, ms, gate, up, n, sinter, limit, st), "shared mid FP8 launch");
    if (ys && enqueue_gemm(ys, 0, mq, ms, n, &sh->w2, sfmt, st)) return -1;
    return 0;
}

/* The prefill MoE on the block-scaled MFMA: tokens and mid in MXFP8, routed
 * GEMMs on FP4 x FP8, k-order combine. The shared expert runs on the side
 * stream: an FP8 one as the reference's GPU prefill runs it, through the FP8
 * GEMM with the 1x128 activation quantization (w1 and w3, SwiGLU and mid's
 * quantization in one pass, w2; src/80_prefill/dsv4_prefill_moe.c:40-58 over
 * dsv4_prefill_proj.c:17-27), an FP4 one on the exact fp16 path. */
static int enqueue_moe_grouped_mx(float *out, const float *x, int n, const DSV4ExpertW *table,
                           int n_experts, const int *idx, const float *w, int topk,
                           const DSV4ExpertW *shared, int sfmt, int sinter, int hidden, int inter,
                           float limit, hipStream_t st)
{
    const long P = (long)n * topk;
    const int trows = grouped_mx_rows_per_tile();
    if ((size_t)P * inter >= (1u << 31) || (size_t)n * hidden >= (1u << 31) ||
        (size_t)inter * hidden / 2 >= (1u << 31))
        return fail("moe_grouped_mx_dev: %ld pairs x %d / %d tokens x %d exceed 31-bit offsets",
                    P, inter, n, hidden);
    size_t off = 0;
    auto take = [&](size_t b) { const size_t o = off; off += (b + 255) & ~(size_t)255; return o; };
    const long max_tiles = (P + trows - 1) / trows + n_experts;
    const size_t o_grp = take((size_t)(n_experts + 1) * 4), o_tp = take((size_t)(n_experts + 1) * 4);
    const size_t o_tg = take((size_t)(max_tiles + 4) * sizeof(TileRec));
    const size_t o_pos = take((size_t)P * 4), o_row = take((size_t)P * 4);
    const size_t o_ch = take(route_chist_bytes(P, n_experts));
    const size_t o_x8 = take((size_t)n * hidden), o_xs = take((size_t)n * hidden / 32);
    const size_t o_mid = take((size_t)P * inter), o_ms = take((size_t)P * inter / 32);
    const size_t o_y = take((size_t)P * hidden * 4);
    const bool sh_fp8 = shared && (sfmt == FMT_FP8_E8M0 || sfmt == FMT_FP8_F32S);
    size_t o_x16 = 0, o_ex = 0, o_smid = 0, o_ys = 0;
    size_t o_sxq = 0, o_sxs = 0, o_sg = 0, o_su = 0, o_smq = 0, o_sms = 0;
    if (sh_fp8) {
        o_sxq = take((size_t)n * hidden);
        o_sxs = take((size_t)n * (hidden / 128) * 4);
        o_sg = take((size_t)n * sinter * 4);
        o_su = take((size_t)n * sinter * 4);
        o_smq = take((size_t)n * sinter);
        o_sms = take((size_t)n * (sinter / 128) * 4);
        o_ys = take((size_t)n * hidden * 4);
    } else if (shared) {
        o_x16 = take((size_t)n * hidden * 2);
        o_ex = take((size_t)n * 4);
        o_smid = take((size_t)n * sinter * 2);
        o_ys = take((size_t)n * hidden * 4);
    }
    HIPCHK(g.moe_ws.need(off), "grouped MoE workspace");
    uint8_t *ws = (uint8_t *)g.moe_ws.p;
    int *grp = (int *)(ws + o_grp), *tp = (int *)(ws + o_tp);
    TileRec *tg = (TileRec *)(ws + o_tg);
    int *pos = (int *)(ws + o_pos), *row = (int *)(ws + o_row);
    uint8_t *x8 = ws + o_x8, *xs = ws + o_xs, *mid = ws + o_mid, *ms = ws + o_ms;
    float *y = (float *)(ws + o_y);

    /* x to MXFP8 on the side stream, beside the routing permutation on this
     * one (neither reads the other's output); the shared expert follows it
     * there */
    HIPCHK(hipEventRecord(g.fork, st), "fork record");
    HIPCHK(hipStreamWaitEvent(g.side, g.fork, 0), "fork wait");
    HIPCHK(quant_act_mxfp8_launch(x8, xs, x, n, hidden, g.side), "x MXFP8 launch");
    HIPCHK(hipEventRecord(g.xq, g.side), "quant record");

    RouteArgs ra;
    ra.idx = idx; ra.npairs = (int)P; ra.topk = topk; ra.n_experts = n_experts;
    ra.tile_rows = trows; ra.grp_off = grp; ra.tile_pre = tp; ra.tile_rec = tg; ra.pos = pos;
    ra.row_tok = row;
    ra.row_k = nullptr;
    ra.chist = (int *)(ws + o_ch);
    ra.status = g.st;
    HIPCHK(moe_route_launch(ra, st), "route launch");

    float *ys = nullptr;
    if (sh_fp8) {
        ys = (float *)(ws + o_ys);
        if (enqueue_shared_fp8q(ys, ws + o_smq, (float *)(ws + o_sms), x, n, shared, sfmt, sinter, hidden, limit,
                                ws + o_sxq, (float *)(ws + o_sxs), (float *)(ws + o_sg), (float *)(ws + o_su),
                                g.side))
            return -1;
        HIPCHK(hipEventRecord(g.join, g.side), "join record");
    } else if (shared) {
        /* an FP4 shared expert on the side stream: its own fp16 copy of x */
        uint16_t *x16 = (uint16_t *)(ws + o_x16), *smid = (uint16_t *)(ws + o_smid);
        int *ex = (int *)(ws + o_ex);
        ys = (float *)(ws + o_ys);
        HIPCHK(to_f16_rows_launch(x16, ex, x, n, hidden, g.side), "shared x fp16 launch");
        const int stt = n <= 64 ? 1 : 4;
        const long stiles = (n + grouped_rows_per_tile(stt) - 1) / grouped_rows_per_tile(stt);
        GroupedArgs sa;
        memset(&sa, 0, sizeof sa);
        sa.m1 = shared->w1; sa.m3 = shared->w3; sa.nrows = n; sa.B = x16; sa.bexp = ex;
        sa.K = hidden; sa.N = sinter; sa.out = smid; sa.limit = limit; sa.status = g.st;
        HIPCHK(grouped_launch(sfmt, true, stt, sa, stiles, g.side), "shared gate/up launch");
        sa.m1 = shared->w2; sa.B = smid; sa.bexp = nullptr; sa.K = sinter; sa.N = hidden; sa.out = ys;
        HIPCHK(grouped_launch(sfmt, false, stt, sa, stiles, g.side), "shared down launch");
        HIPCHK(hipEventRecord(g.join, g.side), "join record");
    }

    HIPCHK(hipStreamWaitEvent(st, g.xq, 0), "quant wait");
    GroupedMxArgs ga;
    memset(&ga, 0, sizeof ga);
    ga.table = table; ga.n_experts = n_experts; ga.grp_off = grp; ga.tile_pre = tp; ga.tile_rec = tg;
    ga.row_tok = row; ga.B = x8; ga.BS = xs; ga.nrows = n; ga.K = hidden; ga.N = inter;
    ga.out = mid; ga.out_s = ms; ga.limit = limit; ga.status = g.st;
    /* thin tiles (weight streaming) on a second side stream, beside the fat
     * tiles (MFMA) on this one; each down launch reads only mid rows its own
     * gate/up launch wrote */
    HIPCHK(hipEventRecord(g.fork2, st), "fork record");
    HIPCHK(hipStreamWaitEvent(g.side2, g.fork2, 0), "fork wait");
    HIPCHK(grouped_mx_launch(true, ga, max_tiles, st, g.side2), "routed gate/up launch");
    ga.row_tok = nullptr; ga.B = mid; ga.BS = ms; ga.nrows = (int)P; ga.K = inter; ga.N = hidden;
    ga.out = y; ga.out_s = nullptr;
    HIPCHK(grouped_mx_launch(false, ga, max_tiles, st, g.side2), "routed down launch");
    HIPCHK(hipEventRecord(g.join2, g.side2), "join record");
    HIPCHK(hipStreamWaitEvent(st, g.join2, 0), "join wait");

    if (shared) HIPCHK(hipStreamWaitEvent(st, g.join, 0), "join wait");
    CombineArgs ca;
    ca.out = out; ca.Y = y; ca.YS = ys; ca.w = w; ca.pos = pos;
    ca.n = n; ca.topk = topk; ca.hidden = hidden;
    HIPCHK(moe_combine_launch(ca, st), "combine launch");
    return 0;
}

/* Checks shared by both grouped entry points; returns the shared format. */
static int grouped_checks(int n, int topk, int n_experts, int hidden, int inter,
                   const DSV4ExpertW *shared, int *sfmt, int *sinter, const char *what)
{
    if (n < 1) return fail("%s: n %d < 1", what, n);
    if (topk < 1 || topk > 16) return fail("%s: topk %d outside 1..16", what, topk);
    if (n_experts < 1 || n_experts > 1024) return fail("%s: n_experts %d outside 1..1024", what, n_experts);
    if (hidden <= 0 || inter <= 0 || hidden % 128 || inter % 128)
        return fail("%s: hidden %d and inter %d must be multiples of 128", what, hidden, inter);
    if ((long)n * topk > (1L << 26)) return fail("%s: %d x %d pairs is too many", what, n, topk);
    *sfmt = -1;
    *sinter = 0;
    if (shared) {
        int sh;
        if (expert_geometry(shared, sfmt, sinter, &sh, what)) return -1;
        if (sh != hidden) return fail("%s: shared hidden %d != %d", what, sh, hidden);
        if (*sinter % 128) return fail("%s: shared inter %d is not a multiple of 128", what, *sinter);
        if (*sfmt == FMT_FP8_E8M0 || *sfmt == FMT_FP8_F32S) {
            if (shared->w1.blk_r != 128 || shared->w3.blk_r != 128 || shared->w2.blk_r != 128)
                return fail("%s: shared FP8 needs 128x128 scale blocks", what);
        } else if (shared->w1.blk_r != 1 || shared->w3.blk_r != 1 || shared->w2.blk_r != 1) {
            return fail("%s: shared FP4 needs 1x32 scale blocks", what);
        }
        const DSV4QMat *ms[3] = {&shared->w1, &shared->w3, &shared->w2};
        for (int i = 0; i < 3; i++)
            if (!aligned16(ms[i]->w) || ((uintptr_t)ms[i]->s & 3u))
                return fail("%s: shared weights must be 16-byte and scales 4-byte aligned", what);
    }
    return 0;
}

int dsv4_hip_moe_grouped_dev(float *out, const float *x, int n, const DSV4ExpertW *experts,
                             int n_experts, const int *idx, const float *w, int topk,
                             const DSV4ExpertW *shared, int hidden, int inter, float limit,
                             void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_grouped_dev");
    if (usable()) return -1;
    dev_call();
    if (!out || !x || !experts || !idx || !w) return fail("moe_grouped_dev: NULL pointer");
    int sfmt, sinter;
    if (grouped_checks(n, topk, n_experts, hidden, inter, shared, &sfmt, &sinter, "moe_grouped_dev"))
        return -1;
    if (!aligned16(x) || !aligned16(out)) return fail("moe_grouped_dev: x and out must be 16-byte aligned");
    return enqueue_moe_grouped(out, x, n, experts, n_experts, idx, w, topk, shared, sfmt, sinter,
                               hidden, inter, limit, (hipStream_t)stream);
}

int dsv4_hip_moe_layer_n_dev(float *out, const float *x, int n, const DSV4QMat *gate,
                             const float *bias, const int64_t *tid2eid, int n_vocab,
                             const int *token_ids, float route_scale,
                             const DSV4ExpertW *experts, int n_experts, int topk,
                             const DSV4ExpertW *shared, int hidden, int inter, float limit, int mx,
                             int *idx_out, float *w_out, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_layer_n_dev");
    if (usable()) return -1;
    dev_call();
    const char *what = "moe_layer_n_dev";
    if (n <= 0) return fail("%s: n %d < 1", what, n);
    if (!out || !x || !experts) return fail("%s: NULL pointer", what);
    int gfmt, sfmt, sinter;
    if (check_qmat(gate, "moe_layer_n_dev gate", &gfmt)) return -1;
    if (!gate->w || (gfmt != FMT_BF16 && !gate->s)) return fail("%s: NULL gate pointer", what);
    if (gate->rows != n_experts || gate->cols != hidden)
        return fail("%s: gate is [%d x %d], expected [%d x %d]", what, gate->rows, gate->cols,
                    n_experts, hidden);
    if (!aligned16(gate->w)) return fail("%s: gate weights must be 16-byte aligned", what);
    if (route_checks(what, n_experts, topk, tid2eid, n_vocab)) return -1;
    if (tid2eid && !token_ids) return fail("%s: hash routing needs token_ids", what);
    if (grouped_checks(n, topk, n_experts, hidden, inter, shared, &sfmt, &sinter, what)) return -1;
    if (mx && hidden % 256) return fail("%s: hidden %d is not a multiple of 256", what, hidden);
    if (!aligned16(x) || !aligned16(out)) return fail("%s: x and out must be 16-byte aligned", what);
    const hipStream_t st = (hipStream_t)stream;
    const size_t sb = ((size_t)n * n_experts * 4 + 255) & ~(size_t)255;
    const size_t rb = ((size_t)n * topk * 4 + 255) & ~(size_t)255;
    HIPCHK(g.route.need(sb + 2 * rb), "router workspace");
    float *scores = (float *)g.route.p;
    int *idx = idx_out ? idx_out : (int *)((uint8_t *)g.route.p + sb);
    float *w = w_out ? w_out : (float *)((uint8_t *)g.route.p + sb + rb);
    if (enqueue_mmq(*gate, gfmt, x, scores, n, st)) return -1;
    GateRouteArgs a;
    memset(&a, 0, sizeof a);
    a.scores = scores;
    a.scores_ld = n_experts;
    a.n = n;
    a.bias = bias;
    a.tid2eid = tid2eid;
    a.n_vocab = n_vocab;
    a.token_ids = token_ids;
    a.n_experts = n_experts;
    a.topk = topk;
    a.route_scale = route_scale;
    a.idx = idx;
    a.w = w;
    a.status = g.st;
    HIPCHK(gate_route_launch(a, st), "route launch");
    return mx ? enqueue_moe_grouped_mx(out, x, n, experts, n_experts, idx, w, topk, shared, sfmt, sinter,
                                       hidden, inter, limit, st)
              : enqueue_moe_grouped(out, x, n, experts, n_experts, idx, w, topk, shared, sfmt, sinter,
                                    hidden, inter, limit, st);
}

int dsv4_hip_moe_grouped_mx_dev(float *out, const float *x, int n, const DSV4ExpertW *experts,
                                int n_experts, const int *idx, const float *w, int topk,
                                const DSV4ExpertW *shared, int hidden, int inter, float limit,
                                void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_grouped_mx_dev");
    if (usable()) return -1;
    dev_call();
    if (!out || !x || !experts || !idx || !w) return fail("moe_grouped_mx_dev: NULL pointer");
    int sfmt, sinter;
    if (grouped_checks(n, topk, n_experts, hidden, inter, shared, &sfmt, &sinter,
                       "moe_grouped_mx_dev"))
        return -1;
    if (hidden % 256) return fail("moe_grouped_mx_dev: hidden %d is not a multiple of 256", hidden);
    if (!aligned16(x) || !aligned16(out))
        return fail("moe_grouped_mx_dev: x and out must be 16-byte aligned");
    return enqueue_moe_grouped_mx(out, x, n, experts, n_experts, idx, w, topk, shared, sfmt, sinter,
                                  hidden, inter, limit, (hipStream_t)stream);
}

int dsv4_hip_moe_grouped_mx_mid_dev(uint8_t *mid, uint8_t *mid_s, int *row_tok, int *row_k,
                                    const float *x, int n, const DSV4ExpertW *experts,
                                    int n_experts, const int *idx, int topk, int hidden, int inter,
                                    float limit, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_grouped_mx_mid_dev");
    if (usable()) return -1;
    dev_call();
    if (!mid || !mid_s || !row_tok || !row_k || !x || !experts || !idx)
        return fail("moe_grouped_mx_mid_dev: NULL pointer");
    int sfmt, sinter;
    if (grouped_checks(n, topk, n_experts, hidden, inter, nullptr, &sfmt, &sinter,
                       "moe_grouped_mx_mid_dev"))
        return -1;
    if (!aligned16(x) || ((uintptr_t)mid & 3) || ((uintptr_t)mid_s & 3))
        return fail("moe_grouped_mx_mid_dev: x 16-byte, mid and mid_s 4-byte aligned");
    const long P = (long)n * topk;
    if ((size_t)P * inter >= (1u << 31) || (size_t)n * hidden >= (1u << 31))
        return fail("moe_grouped_mx_mid_dev: too many pairs or tokens for 31-bit offsets");
    hipStream_t st = (hipStream_t)stream;
    const int trows = grouped_mx_rows_per_tile();
    const long max_tiles = (P + trows - 1) / trows + n_experts;
    size_t off = 0;
    auto take = [&](size_t b) { const size_t o = off; off += (b + 255) & ~(size_t)255; return o; };
    const size_t o_grp = take((size_t)(n_experts + 1) * 4), o_tp = take((size_t)(n_experts + 1) * 4);
    const size_t o_tg = take((size_t)(max_tiles + 4) * sizeof(TileRec)), o_pos = take((size_t)P * 4);
    const size_t o_ch = take(route_chist_bytes(P, n_experts));
    const size_t o_x8 = take((size_t)n * hidden), o_xs = take((size_t)n * hidden / 32);
    HIPCHK(g.moe_ws.need(off), "grouped MoE workspace");
    uint8_t *ws = (uint8_t *)g.moe_ws.p;
    RouteArgs ra;
    ra.idx = idx; ra.npairs = (int)P; ra.topk = topk; ra.n_experts = n_experts; ra.tile_rows = trows;
    ra.grp_off = (int *)(ws + o_grp); ra.tile_pre = (int *)(ws + o_tp); ra.tile_rec = (TileRec *)(ws + o_tg);
    ra.pos = (int *)(ws + o_pos); ra.row_tok = row_tok; ra.row_k = row_k; ra.status = g.st;
    ra.chist = (int *)(ws + o_ch);
    HIPCHK(moe_route_launch(ra, st), "route launch");
    HIPCHK(quant_act_mxfp8_launch(ws + o_x8, ws + o_xs, x, n, hidden, st), "x MXFP8 launch");
    GroupedMxArgs ga;
    memset(&ga, 0, sizeof ga);
    ga.table = experts; ga.n_experts = n_experts; ga.grp_off = ra.grp_off; ga.tile_pre = ra.tile_pre;
    ga.tile_rec = ra.tile_rec; ga.row_tok = row_tok; ga.B = ws + o_x8; ga.BS = ws + o_xs; ga.nrows = n;
    ga.K = hidden; ga.N = inter; ga.out = mid; ga.out_s = mid_s; ga.limit = limit; ga.status = g.st;
    HIPCHK(grouped_mx_launch(true, ga, max_tiles, st, st), "routed gate/up launch");
    return 0;
}

int dsv4_hip_shared_fp8q_mid_dev(uint8_t *mid, float *mid_s, const float *x, int n,
                                 const DSV4ExpertW *shared, int hidden, float limit, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_shared_fp8q_mid_dev");
    if (usable()) return -1;
    dev_call();
    const char *what = "shared_fp8q_mid_dev";
    if (!mid || !mid_s || !x || !shared) return fail("%s: NULL pointer", what);
    if (!aligned16(x) || ((uintptr_t)mid & 7u)) return fail("%s: x must be 16- and mid 8-byte aligned", what);
    int sfmt, sinter;
    if (grouped_checks(n, 1, 1, hidden, 128, shared, &sfmt, &sinter, what)) return -1;
    if (sfmt != FMT_FP8_E8M0 && sfmt != FMT_FP8_F32S) return fail("%s: the shared expert must be FP8", what);
    if ((size_t)n * hidden >= (1u << 31) || (size_t)n * sinter >= (1u << 31))
        return fail("%s: %d tokens exceed 31-bit offsets", what, n);
    size_t off = 0;
    auto take = [&](size_t b) { const size_t o = off; off += (b + 255) & ~(size_t)255; return o; };
    const size_t o_xq = take((size_t)n * hidden), o_xs = take((size_t)n * (hidden / 128) * 4);
    const size_t o_g = take((size_t)n * sinter * 4), o_u = take((size_t)n * sinter * 4);
    HIPCHK(g.moe_ws.need(off), "shared workspace");
    uint8_t *ws = (uint8_t *)g.moe_ws.p;
    return enqueue_shared_fp8q(nullptr, mid, mid_s, x, n, shared, sfmt, sinter, hidden, limit, ws + o_xq,
                               (float *)(ws + o_xs), (float *)(ws + o_g), (float *)(ws + o_u),
                               (hipStream_t)stream);
}

int dsv4_hip_moe_grouped(float *out, const float *x, int n, const int *topk_idx,
                         const float *topk_w, int topk, const DSV4ExpertW *experts,
                         int n_experts, const DSV4ExpertW *shared, float limit)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_grouped");
    if (usable()) return -1;
    if (!out || !x || !topk_idx || !topk_w || !experts) return fail("moe_grouped: NULL pointer");
    if (n_experts < 1 || n_experts > 1024) return fail("moe_grouped: n_experts %d outside 1..1024", n_experts);
    std::vector<DSV4ExpertW> tab((size_t)n_experts);
    int inter = 0, hidden = 0;
    for (int e = 0; e < n_experts; e++) {
        int fmt, ei, eh;
        if (expert_geometry(&experts[e], &fmt, &ei, &eh, "moe_grouped routed")) return -1;
        if (fmt != FMT_FP4_E8M0 || experts[e].w1.blk_r != 1)
            return fail("moe_grouped: routed expert %d is not FP4 with 1x32 scales", e);
        if (e == 0) { inter = ei; hidden = eh; }
        else if (ei != inter || eh != hidden) return fail("moe_grouped: routed shapes differ (expert %d)", e);
        if (resident_expert(&experts[e], &tab[(size_t)e], "moe_grouped routed")) return -1;
    }
    DSV4ExpertW sdev;
    int sfmt, sinter;
    if (shared && resident_expert(shared, &sdev, "moe_grouped shared")) return -1;
    if (grouped_checks(n, topk, n_experts, hidden, inter, shared ? &sdev : nullptr, &sfmt, &sinter,
                       "moe_grouped"))
        return -1;
    host_call();
    const size_t P = (size_t)n * topk;
    const size_t tb = ((size_t)n_experts * sizeof(DSV4ExpertW) + 255) & ~(size_t)255;
    const size_t ib = (P * 4 + 255) & ~(size_t)255;
    HIPCHK(g.table.need(tb + 2 * ib), "table alloc");
    HIPCHK(g.x.need((size_t)n * hidden * 4), "x staging");
    HIPCHK(g.y.need((size_t)n * hidden * 4), "out staging");
    uint8_t *tp = (uint8_t *)g.table.p;
    HIPCHK(hipMemcpyAsync(tp, tab.data(), (size_t)n_experts * sizeof(DSV4ExpertW), hipMemcpyHostToDevice, g.stream), "table upload");
    HIPCHK(hipMemcpyAsync(tp + tb, topk_idx, P * 4, hipMemcpyHostToDevice, g.stream), "routing upload");
    HIPCHK(hipMemcpyAsync(tp + tb + ib, topk_w, P * 4, hipMemcpyHostToDevice, g.stream), "weights upload");
    HIPCHK(hipMemcpyAsync(g.x.p, x, (size_t)n * hidden * 4, hipMemcpyHostToDevice, g.stream), "x upload");
    if (enqueue_moe_grouped((float *)g.y.p, (const float *)g.x.p, n, (const DSV4ExpertW *)tp,
                            n_experts, (const int *)(tp + tb), (const float *)(tp + tb + ib), topk,
                            shared ? &sdev : nullptr, sfmt, sinter, hidden, inter, limit, g.stream))
        return -1;
    HIPCHK(hipMemcpyAsync(out, g.y.p, (size_t)n * hidden * 4, hipMemcpyDeviceToHost, g.stream), "out download");
    return finish_host_call("moe_grouped");
}

int dsv4_hip_moe_route_dev(int *ex_off, int *ex_tok, int *ex_k, int *pos, const int *idx, int n,
                           int topk, int n_experts, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_moe_route_dev");
    if (usable()) return -1;
    dev_call();
    if (!ex_off || !ex_tok || !ex_k || !pos || !idx) return fail("moe_route_dev: NULL pointer");
    if (n < 1 || topk < 1 || topk > 16 || (long)n * topk > (1L << 26))
        return fail("moe_route_dev: bad n %d / topk %d", n, topk);
    if (n_experts < 1 || n_experts > 1024)
        return fail("moe_route_dev: n_experts %d outside 1..1024", n_experts);
    const long P = (long)n * topk;
    const int trows = 16;
    const long max_tiles = (P + trows - 1) / trows + n_experts;
    const size_t o_tp = 0, o_tg = (((size_t)n_experts + 1) * 4 + 255) & ~(size_t)255;
    const size_t o_ch = (o_tg + (size_t)(max_tiles + 4) * sizeof(TileRec) + 255) & ~(size_t)255;
    HIPCHK(g.small.need(o_ch + route_chist_bytes(P, n_experts)), "route workspace");
    RouteArgs ra;
    ra.idx = idx; ra.npairs = (int)P; ra.topk = topk; ra.n_experts = n_experts;
    ra.tile_rows = trows; ra.grp_off = ex_off;
    ra.tile_pre = (int *)((uint8_t *)g.small.p + o_tp);
    ra.tile_rec = (TileRec *)((uint8_t *)g.small.p + o_tg);
    ra.pos = pos; ra.row_tok = ex_tok; ra.row_k = ex_k; ra.status = g.st;
    ra.chist = (int *)((uint8_t *)g.small.p + o_ch);
    HIPCHK(moe_route_launch(ra, (hipStream_t)stream), "route launch");
    return 0;
}

int dsv4_hip_status(unsigned *bits)
{
    std::lock_guard<std::mutex> lk(g.mu);
    Range rg("dsv4_hip_status");
    if (!g.ready) return fail("not initialised");
    HIPCHK(hipDeviceSynchronize(), "status sync");
    unsigned v = 0;
    HIPCHK(hipMemcpy(&v, g.status, sizeof v, hipMemcpyDeviceToHost), "status read");
    HIPCHK(hipMemset(g.status, 0, sizeof v), "status clear");
    if (bits) *bits = v;
    return 0;
}

/* ------------------------------------------------------------- aux ---- */

int dsv4_hip_dequant_dev(float *out, const DSV4QMat *m, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (usable()) return -1;
    int fmt;
    if (check_qmat(m, "dequant_dev", &fmt)) return -1;
    if (fmt == FMT_BF16) return fail("dequant_dev: BF16 has no packed format to decode");
    if (!out || !m->w || !m->s) return fail("dequant_dev: NULL pointer");
    if (!aligned16(m->w)) return fail("dequant_dev: W must be 16-byte aligned");
    HIPCHK(dequant_launch(fmt, *m, out, (hipStream_t)stream), "dequant launch");
    return 0;
}

int dsv4_hip_quant_fp8_blk128_dev(uint8_t *W, float *S, const float *w, int rows,
                                  int cols, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (usable()) return -1;
    if (!W || !S || !w || rows <= 0 || cols <= 0) return fail("quant_fp8_blk128_dev: bad argument");
    HIPCHK(quant_fp8_blk128_launch(W, S, w, rows, cols, (hipStream_t)stream), "quant launch");
    return 0;
}

int dsv4_hip_quant_fp4_mx_dev(uint8_t *W, uint8_t *S, const float *w, int rows,
                              int cols, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (usable()) return -1;
    if (!W || !S || !w || rows <= 0 || cols <= 0 || cols % 32)
        return fail("quant_fp4_mx_dev: bad argument");
    if (!aligned16(W) || !aligned16(w)) return fail("quant_fp4_mx_dev: W and w must be 16-byte aligned");
    HIPCHK(quant_fp4_mx_launch(W, S, w, rows, cols, (hipStream_t)stream), "quant launch");
    return 0;
}

int dsv4_hip_quant_act_fp8_1x128_dev(uint8_t *Q, float *S, const float *a, int n,
                                     int k, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (usable()) return -1;
    if (!Q || !S || !a || n <= 0 || k <= 0 || k % 128)
        return fail("quant_act_fp8_1x128_dev: bad argument");
    if (((uintptr_t)Q & 7u) != 0 || ((uintptr_t)a & 15u) != 0 || ((uintptr_t)S & 3u) != 0)
        return fail("quant_act_fp8_1x128_dev: need Q 8-, a 16- and S 4-byte aligned");
    HIPCHK(quant_act_fp8_1x128_launch(Q, S, a, n, k, false, true, (hipStream_t)stream),
           "quant launch");
    return 0;
}

int dsv4_hip_quant_act_mxfp8_dev(uint8_t *Q, uint8_t *S, const float *a, int n,
                                 int k, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (usable()) return -1;
    if (!Q || !S || !a || n <= 0 || k <= 0 || k % 32)
        return fail("quant_act_mxfp8_dev: bad argument");
    if (!aligned16(Q) || !aligned16(a)) return fail("quant_act_mxfp8_dev: Q and a must be 16-byte aligned");
    HIPCHK(quant_act_mxfp8_launch(Q, S, a, n, k, (hipStream_t)stream), "quant launch");
    return 0;
}

int dsv4_hip_synth_normal_dev(float *out, size_t n, uint64_t seed, float sigma,
                              int round_bf16, void *stream)
{
    std::lock_guard<std::mutex> lk(g.mu);
    if (usable()) return -1;
    if (!out || !n) return fail("synth_normal_dev: bad argument");
    HIPCHK(synth_normal_launch(out, n, seed, sigma, round_bf16, (hipStream_t)stream), "synth launch");
    return 0;
}

} // extern "C"
