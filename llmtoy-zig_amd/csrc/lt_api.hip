// lt_api.hip -- the C ABI (include/llmtoy_hip.h): contexts, tensor upload
// into the planar device layout, argument validation, and kernel dispatch.
#include "llmtoy_hip.h"
#include "lt_internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <new>
#include <string>
#include <vector>

using lt::DevTensor;

struct lt_tensor {
    DevTensor t;
};

namespace {

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

// LT_PROFILE state: event spans around each call's device work (the
// counterpart of the reference's GpuProfiler, gpu/context.zig:34-268) and,
// with LT_PROFILE=timeline, the single-launch MoE kernel's phase stamps.
struct PendingSpan {
    hipEvent_t a, b;
    const char *label;
};
struct SpanStat {
    size_t n = 0;
    double total_ms = 0, min_ms = 1e30, max_ms = 0;
};
constexpr int kRoles = 8, kPhases = lt::kStamps - 1;
struct Profile {
    int mode = 0;  // 0 off, 1 spans, 2 spans + timeline
    std::vector<PendingSpan> pending;
    std::vector<hipEvent_t> free_events;
    std::map<std::string, SpanStat> spans;
    uint64_t *stamps = nullptr;  // device [kFusedBlocks][kStamps]
    bool stamps_pending = false;
    size_t launches = 0;
    // per launch: median and largest time of each (role, phase) over blocks, us
    std::vector<float> med[kRoles][kPhases], last[kRoles][kPhases];
    std::string placement;  // CU placement of XCD group 0's blocks in the first harvested launch
    std::vector<float> slot_last[2][16];  // per slot: gate/up h published, down adds issued
    std::vector<float> last_stamp;        // per launch: the last stamp of any block, us
    size_t split = 0;                     // launches with a group (bid % 8) spread over XCDs
    size_t rot[8] = {};                   // launches by XCD of block 0
};

}  // namespace

struct lt_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    // context-owned device scratch, grown on demand
    DevBuf x, out, logits, h, ids, w, shared, g, u, ids_io, w_io, bias, eh, pf, nrm, sink;
    // buffers replaced by larger ones; a HIP graph captured earlier may still
    // reference them, so they are released only by lt_destroy
    std::vector<void *> retired;
    // arrival ticket of the router's last-block top-k; zeroed once at init,
    // every launch leaves it at zero again
    unsigned *ticket = nullptr;
    // hand-over memory of the fused MoE kernel (allocated on first use); the
    // host-mapped error word it reports timed-out waits in (set up by
    // lt_init, with err_dev its device address); whether blocks with equal
    // index % 8 share an XCD (probed by lt_init)
    void *fused = nullptr;
    uint32_t *fused_err = nullptr;
    uint32_t *err_dev = nullptr;
    int xcd_local = 0;
    lt::FusedScratch fsc{};
    // the library's static scratch on this device (lt_noalloc.hip), used by
    // lt_moe_forward_noalloc
    uint8_t *na_base = nullptr;
    lt::FusedScratch na_fsc{};
    // hand-over memory of the single-launch dense FFN (allocated by lt_init)
    void *ffn = nullptr;
    lt::FfnScratch ffsc{};
    Profile prof;
    // pinned + device staging of tensor uploads and read-backs (allocated on first use)
    lt::UploadStaging up{};
};

namespace {

int fail(lt_ctx *ctx, int code, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return code;
}

int hip_fail(lt_ctx *ctx, hipError_t e, const char *what) {
    return fail(ctx, e == hipErrorOutOfMemory ? LT_ERR_OOM : LT_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define LT_HIP(ctx, call)                                     \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
    } while (0)

// Context scratch of at least `bytes`.  A buffer is never freed before
// lt_destroy: a call captured into a HIP graph keeps the scratch addresses
// it was captured with, so a larger call later gets a new buffer and the old
// one is retired (kept allocated).  Capacities at least double, which bounds
// the retired bytes by the final capacity.
int ensure(lt_ctx *ctx, DevBuf &b, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (b.cap >= bytes) return LT_OK;
    size_t cap = (bytes + 4095) & ~(size_t)4095;
    if (cap < 2 * b.cap) cap = 2 * b.cap;
    if (b.p) {
        try {
            ctx->retired.reserve(ctx->retired.size() + 1);  // so that push_back below cannot throw
        } catch (...) {
            return fail(ctx, LT_ERR_OOM, "host allocation failed");
        }
    }
    void *p = nullptr;
    LT_HIP(ctx, hipMalloc(&p, cap));
    if (b.p) ctx->retired.push_back(b.p);
    b.p = p;
    b.cap = cap;
    return LT_OK;
}

// True while the context's stream is being captured into a graph.
bool capturing(lt_ctx *ctx) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(ctx->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// An event pair around the device work one call enqueues (LT_PROFILE set;
// not while the stream is being captured).  Resolved by prof_harvest.
struct Span {
    lt_ctx *ctx = nullptr;
    hipEvent_t a = nullptr;
    const char *label;
    Span(lt_ctx *c, const char *l) : label(l) {
        if (!c->prof.mode || capturing(c)) return;
        Profile &P = c->prof;
        hipEvent_t e = nullptr;
        if (!P.free_events.empty()) {
            e = P.free_events.back();
            P.free_events.pop_back();
        } else if (hipEventCreate(&e) != hipSuccess) {
            return;
        }
        if (hipEventRecord(e, c->stream) != hipSuccess) {
            P.free_events.push_back(e);
            return;
        }
        ctx = c;
        a = e;
    }
    ~Span() {
        if (!ctx) return;
        Profile &P = ctx->prof;
        hipEvent_t b = nullptr;
        if (!P.free_events.empty()) {
            b = P.free_events.back();
            P.free_events.pop_back();
        } else if (hipEventCreate(&b) != hipSuccess) {
            P.free_events.push_back(a);
            return;
        }
        if (hipEventRecord(b, ctx->stream) != hipSuccess) {
            P.free_events.push_back(a);
            P.free_events.push_back(b);
            return;
        }
        P.pending.push_back({a, b, label});
    }
};

float median_of(std::vector<float> v) {
    if (v.empty()) return 0.0f;
    std::nth_element(v.begin(), v.begin() + v.size() / 2, v.end());
    return v[v.size() / 2];
}

// After the stream is idle: resolves pending spans and, with a fused launch
// since the last harvest, reads its phase stamps and adds that launch's
// per-phase medians and maxima (us from the first block's start).
void prof_harvest(lt_ctx *ctx) {
    Profile &P = ctx->prof;
    if (!P.mode) return;
    for (const PendingSpan &sp : P.pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, sp.a, sp.b) == hipSuccess) {
            SpanStat &st = P.spans[sp.label];
            st.n++;
            st.total_ms += ms;
            st.min_ms = std::min(st.min_ms, (double)ms);
            st.max_ms = std::max(st.max_ms, (double)ms);
        }
        P.free_events.push_back(sp.a);
        P.free_events.push_back(sp.b);
    }
    P.pending.clear();
    if (!P.stamps || !P.stamps_pending) return;
    P.stamps_pending = false;
    std::vector<uint64_t> st((size_t)lt::kFusedBlocks * lt::kStamps);
    if (hipMemcpy(st.data(), P.stamps, st.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) return;
    uint64_t t0 = ~0ull;
    for (int b = 0; b < lt::kFusedBlocks; b++) {
        const uint64_t *t = &st[(size_t)b * lt::kStamps];
        if ((t[lt::kStamps - 1] & 0xff) && t[0]) t0 = std::min(t0, t[0]);
    }
    if (t0 == ~0ull) return;
    std::vector<float> v[kRoles][kPhases];
    std::vector<float> sl[2][16];
    uint64_t tmax = t0;
    bool split = false;
    for (int b = 0; b < lt::kFusedBlocks; b++) {
        const uint64_t w = st[(size_t)b * lt::kStamps + lt::kStamps - 1], w0 = st[(size_t)(b & 7) * lt::kStamps + lt::kStamps - 1];
        split |= ((w >> 16) & 15) != ((w0 >> 16) & 15);
    }
    P.split += split;
    P.rot[(st[lt::kStamps - 1] >> 16) & 7]++;
    for (int b = 0; b < lt::kFusedBlocks; b++) {
        const uint64_t *t = &st[(size_t)b * lt::kStamps];
        const int role = (int)(t[lt::kStamps - 1] & 0xff), slot = (int)((t[lt::kStamps - 1] >> 8) & 15);
        if (role <= 0 || role >= kRoles) continue;
        for (int ph = 0; ph < kPhases; ph++)
            if (t[ph] >= t0) {
                v[role][ph].push_back((float)(t[ph] - t0) * 0.01f);  // 100 MHz ticks -> us
                tmax = std::max(tmax, t[ph]);
            }
        if ((role == 2 || role == 3) && t[4] >= t0) sl[role - 2][slot].push_back((float)(t[4] - t0) * 0.01f);
    }
    for (int r = 0; r < kRoles; r++)
        for (int ph = 0; ph < kPhases; ph++) {
            if (v[r][ph].empty()) continue;
            P.med[r][ph].push_back(median_of(v[r][ph]));
            P.last[r][ph].push_back(*std::max_element(v[r][ph].begin(), v[r][ph].end()));
        }
    for (int r = 0; r < 2; r++)
        for (int q = 0; q < 16; q++)
            if (!sl[r][q].empty()) P.slot_last[r][q].push_back(*std::max_element(sl[r][q].begin(), sl[r][q].end()));
    P.last_stamp.push_back((float)(tmax - t0) * 0.01f);
    if (P.placement.empty()) {
        // the first harvested launch: which in-group indices (block / 8) of
        // XCD group 0 shared a CU (HW_ID bits 8-15: CU, shader array,
        // engine), with their roles
        static const char rc[] = "-RGDCsdT";
        std::map<uint32_t, std::string> cu;
        for (int b = 0; b < lt::kFusedBlocks; b += 8) {
            const uint64_t w = st[(size_t)b * lt::kStamps + lt::kStamps - 1];
            const int role = (int)(w & 0xff);
            char item[24];
            snprintf(item, sizeof item, " %d%c", b >> 3, role >= 0 && role < 8 ? rc[role] : '?');
            cu[(uint32_t)(w >> 40) & 0xffu] += item;
        }
        P.placement = "placement, XCD group 0, one launch (in-group index + role: R router, G gate/up, D down, "
                      "C combine, s shared gate/up, d shared down, - none), blocks per CU:\n";
        for (const auto &kv : cu) {
            char head[32];
            snprintf(head, sizeof head, "  CU 0x%02x:", kv.first);
            P.placement += head + kv.second + "\n";
        }
    }
    P.launches++;
}

size_t block_elems(uint32_t type) {
    switch (type) {
    case LT_TYPE_F32: return 1;
    case LT_TYPE_Q8_0: return 32;
    case LT_TYPE_Q4_K:
    case LT_TYPE_Q6_K:
    case LT_TYPE_Q3_K: return 256;
    case LT_TYPE_Q5_0:
    case LT_TYPE_Q5_1:
    case LT_TYPE_IQ4_NL: return 32;
    default: return 0;
    }
}

size_t block_bytes(uint32_t type) {
    switch (type) {
    case LT_TYPE_F32: return 4;
    case LT_TYPE_Q8_0: return 34;
    case LT_TYPE_Q4_K: return 144;
    case LT_TYPE_Q6_K: return 210;
    case LT_TYPE_Q5_0: return 22;
    case LT_TYPE_Q5_1: return 24;
    case LT_TYPE_IQ4_NL: return 18;
    case LT_TYPE_Q3_K: return 110;
    default: return 0;
    }
}

// Largest row length the LDS-staged kernels take (x is staged as fp32).
constexpr size_t kMaxQuantCols = 16384;

void set_planes(DevTensor &t) {
    const size_t nblk = t.total_rows * t.blocks_per_row;
    uint8_t *b = t.base;
    t.p0 = b;
    t.p1 = t.p2 = t.p3 = nullptr;
    switch (t.type) {
    case LT_TYPE_Q8_0: t.p1 = b + nblk * 32; break;
    case LT_TYPE_Q4_K: t.p1 = b + nblk * 16; break;
    case LT_TYPE_Q6_K:
        t.p1 = b + nblk * 128;
        t.p2 = t.p1 + nblk * 64;
        t.p3 = t.p2 + nblk * 16;
        break;
    case LT_TYPE_Q5_0:  // qs [16], qh [4], d [2]
        t.p1 = b + nblk * 16;
        t.p2 = t.p1 + nblk * 4;
        break;
    case LT_TYPE_Q5_1:  // qs [16], qh [4], d and m [4]
        t.p1 = b + nblk * 16;
        t.p2 = t.p1 + nblk * 4;
        break;
    case LT_TYPE_IQ4_NL:  // qs [16], d [2]
        t.p1 = b + nblk * 16;
        break;
    case LT_TYPE_Q3_K:  // qs [64], hmask [32], scales [12], d [2]
        t.p1 = b + nblk * 64;
        t.p2 = t.p1 + nblk * 32;
        t.p3 = t.p2 + nblk * 12;
        break;
    default: break;
    }
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Input staging for LT_HOST_IO: copies host data into a context buffer.
int stage_in(lt_ctx *ctx, DevBuf &buf, const void *host, size_t bytes, const void **dev) {
    int rc = ensure(ctx, buf, bytes);
    if (rc) return rc;
    LT_HIP(ctx, hipMemcpyAsync(buf.p, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    *dev = buf.p;
    return LT_OK;
}

int launch_rc(lt_ctx *ctx, hipError_t e, const char *what) {
    if (e == hipSuccess) return LT_OK;
    return fail(ctx, LT_ERR_DEVICE, "%s launch failed: %s", what, hipGetErrorString(e));
}

// Allocates and zeroes the fused kernel's hand-over memory (once).
int ensure_fused(lt_ctx *ctx) {
    if (ctx->fused) return LT_OK;
    // the one-time set-up clears the memory with a synchronous memset
    if (capturing(ctx))
        return fail(ctx, LT_ERR_INVALID,
                    "the first single-launch MoE call on a context cannot be captured into a graph: make one call "
                    "before capturing");
    void *p = nullptr;
    LT_HIP(ctx, hipMalloc(&p, lt::kFusedScratchBytes));
    const hipError_t e = hipMemset(p, 0, lt::kFusedScratchBytes);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(ctx, e, "fused scratch");
    }
    ctx->fused = p;
    ctx->fsc = lt::fused_scratch_at((uint8_t *)p, ctx->err_dev, ctx->xcd_local);
    ctx->fsc.stamps = ctx->prof.stamps;
    return LT_OK;
}

// lt_init's device set-up: the host-mapped error word, the address of this
// device's static scratch, and the XCD placement probe (run once, into the
// static scratch's probe area).  LT_FUSED_AGENT_HANDOVER=1 turns the same-XCD
// hand-over off (testing).
hipError_t init_device_state(lt_ctx *ctx) {
    void *hp = nullptr, *dp = nullptr;
    hipError_t e = hipHostMalloc(&hp, 64, hipHostMallocMapped);
    if (e != hipSuccess) return e;
    memset(hp, 0, 64);
    ctx->fused_err = (uint32_t *)hp;
    if ((e = hipHostGetDevicePointer(&dp, hp, 0)) != hipSuccess) return e;
    ctx->err_dev = (uint32_t *)dp;
    if ((e = lt::noalloc_scratch(ctx->device, &ctx->na_base)) != hipSuccess) return e;
    int local = 0;
    if ((e = lt::probe_xcd_groups((uint32_t *)(ctx->na_base + lt::kFusedXccOff), ctx->stream, &local)) != hipSuccess)
        return e;
    const char *agent = getenv("LT_FUSED_AGENT_HANDOVER");
    if (agent && agent[0] == '1') local = 0;
    ctx->xcd_local = local;
    ctx->na_fsc = lt::fused_scratch_at(ctx->na_base, ctx->err_dev, local);
    if ((e = hipMalloc(&ctx->ffn, lt::kFfnScratchBytes)) != hipSuccess) return e;
    if ((e = hipMemset(ctx->ffn, 0, lt::kFfnScratchBytes)) != hipSuccess) return e;
    ctx->ffsc = lt::ffn_scratch_at((uint8_t *)ctx->ffn, ctx->err_dev, local);
    // LT_PROFILE: "timeline" = spans + phase stamps of the fused kernel;
    // any other non-empty value except "0" = spans
    const char *prof = getenv("LT_PROFILE");
    if (prof && prof[0] && strcmp(prof, "0") != 0) {
        ctx->prof.mode = strcmp(prof, "timeline") == 0 ? 2 : 1;
        if (ctx->prof.mode == 2) {
            const size_t nb = (size_t)lt::kFusedBlocks * lt::kStamps * 8;
            if ((e = hipMalloc((void **)&ctx->prof.stamps, nb)) != hipSuccess) return e;
            if ((e = hipMemset(ctx->prof.stamps, 0, nb)) != hipSuccess) return e;
            ctx->na_fsc.stamps = ctx->prof.stamps;
        }
    }
    return hipSuccess;
}

// A fused-kernel wait that ran into its time limit (the outputs of that
// call are NaN); reported, and cleared, by the next synchronising call.
int check_fused_err(lt_ctx *ctx) {
    if (!ctx->fused_err) return LT_OK;
    const uint32_t v = __atomic_exchange_n(ctx->fused_err, 0u, __ATOMIC_SEQ_CST);
    if (!v) return LT_OK;
    if (v == lt::kErrCodePrefillSat) {
        const uint32_t n = __atomic_exchange_n(ctx->fused_err + lt::kErrPrefillSat, 0u, __ATOMIC_SEQ_CST);
        return fail(ctx, LT_ERR_DEVICE,
                    "batched prefill: %u expert activations between the two GEMMs fell outside f16's range (after "
                    "the row's power-of-two scaling) and saturated at +-65504; the outputs of that call are inexact",
                    n);
    }
    (void)__atomic_exchange_n(ctx->fused_err + lt::kErrPrefillSat, 0u, __ATOMIC_SEQ_CST);
    uint32_t d[5];  // first timed-out wait: block + 1, site, index, tag or count seen, epoch expected
    for (int i = 0; i < 5; i++) d[i] = __atomic_exchange_n(ctx->fused_err + 2 + i, 0u, __ATOMIC_SEQ_CST);
    // Later launches publish h through memory (agent scope) instead of an
    // XCD's L2, in case the placement the one-time probe saw has changed.
    ctx->xcd_local = ctx->fsc.xcd_local = ctx->na_fsc.xcd_local = ctx->ffsc.xcd_local = 0;
    return fail(ctx, LT_ERR_DEVICE,
                "single-launch kernel: a hand-over wait timed out (code 0x%x: 1 gate/up logits, 2 down logits, 4 down "
                "h records, 8 combine, 0x10 shared-FFN logits or last h word, 0x20 shared-FFN h, 0x40 dense-FFN h, "
                "0x80 dense-FFN start values, 0x100 prefill f16 saturation, 0x200 Gemma4 tail, 0x400 prefill chunk "
                "activations; first recorded: block %d, site 0x%x, index %u, saw %u, expected epoch or count %u); "
                "outputs of that call are NaN (prefill: wrong)",
                v, (int)d[0] - 1, d[1], d[2], d[3], d[4]);
}

int matvec_dev(lt_ctx *ctx, const DevTensor &W, const float *x, float *y) {
    hipError_t e;
    switch (W.type) {
    case LT_TYPE_Q4_K: e = lt::launch_matvec_q4k(W, 0, W.total_rows, x, y, ctx->stream); break;
    case LT_TYPE_Q8_0: e = lt::launch_matvec_q8_0(W, x, y, ctx->stream); break;
    case LT_TYPE_Q6_K: e = lt::launch_matvec_q6k(W, x, y, ctx->stream); break;
    case LT_TYPE_F32: e = lt::launch_matvec_f32(W, x, y, ctx->stream); break;
    case LT_TYPE_Q5_0:
    case LT_TYPE_Q5_1:
    case LT_TYPE_IQ4_NL:
    case LT_TYPE_Q3_K: e = lt::launch_matvec_fmt(W, x, y, ctx->stream); break;
    default: return fail(ctx, LT_ERR_UNSUPPORTED, "matvec: unsupported type %u", W.type);
    }
    return launch_rc(ctx, e, "matvec");
}

int check_matvec_tensor(lt_ctx *ctx, const lt_tensor *W) {
    if (!W) return fail(ctx, LT_ERR_INVALID, "null tensor");
    if (W->t.type != LT_TYPE_F32 && W->t.cols > kMaxQuantCols)
        return fail(ctx, LT_ERR_UNSUPPORTED, "row length %zu exceeds %zu", W->t.cols, kMaxQuantCols);
    return LT_OK;
}

}  // namespace

// ------------------------------------------------------------------ lifecycle
extern "C" int lt_init(int device, lt_ctx **out_ctx) {
    if (!out_ctx) return LT_ERR_INVALID;
    *out_ctx = nullptr;
    const char *force = getenv("LT_FORCE_NO_DEVICE");
    if (force && force[0] == '1') return LT_ERR_DEVICE;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || device < 0 || device >= n) return LT_ERR_DEVICE;
    if (hipSetDevice(device) != hipSuccess) return LT_ERR_DEVICE;
    lt_ctx *ctx = new (std::nothrow) lt_ctx();
    if (!ctx) return LT_ERR_OOM;
    ctx->device = device;
    if (hipStreamCreate(&ctx->stream) != hipSuccess) {
        delete ctx;
        return LT_ERR_DEVICE;
    }
    hipError_t e = hipMalloc((void **)&ctx->ticket, 256);
    if (e == hipSuccess) e = hipMemset(ctx->ticket, 0, 256);
    if (e == hipSuccess) e = init_device_state(ctx);
    if (e != hipSuccess) {
        if (ctx->ticket) (void)hipFree(ctx->ticket);
        if (ctx->fused_err) (void)hipHostFree(ctx->fused_err);
        if (ctx->prof.stamps) (void)hipFree(ctx->prof.stamps);
        if (ctx->ffn) (void)hipFree(ctx->ffn);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return e == hipErrorOutOfMemory ? LT_ERR_OOM : LT_ERR_DEVICE;
    }
    *out_ctx = ctx;
    return LT_OK;
}

extern "C" void lt_destroy(lt_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    DevBuf *bufs[] = {&ctx->x, &ctx->out, &ctx->logits, &ctx->h, &ctx->ids, &ctx->w,
                      &ctx->shared, &ctx->g, &ctx->u, &ctx->ids_io, &ctx->w_io, &ctx->bias, &ctx->eh, &ctx->pf,
                      &ctx->nrm, &ctx->sink};
    for (DevBuf *b : bufs)
        if (b->p) (void)hipFree(b->p);
    for (void *p : ctx->retired) (void)hipFree(p);
    for (const PendingSpan &sp : ctx->prof.pending) {
        (void)hipEventDestroy(sp.a);
        (void)hipEventDestroy(sp.b);
    }
    for (hipEvent_t e : ctx->prof.free_events) (void)hipEventDestroy(e);
    if (ctx->prof.stamps) (void)hipFree(ctx->prof.stamps);
    if (ctx->ticket) (void)hipFree(ctx->ticket);
    if (ctx->fused) (void)hipFree(ctx->fused);
    if (ctx->ffn) (void)hipFree(ctx->ffn);
    if (ctx->fused_err) (void)hipHostFree(ctx->fused_err);
    lt::free_staging(ctx->up);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

extern "C" const char *lt_last_error(const lt_ctx *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

extern "C" int lt_sync(lt_ctx *ctx) {
    if (!ctx) return LT_ERR_INVALID;
    LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    prof_harvest(ctx);
    return check_fused_err(ctx);
}

extern "C" void *lt_stream(lt_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

// ------------------------------------------------------------------ tensors
extern "C" int lt_tensor_upload(lt_ctx *ctx, const void *host_bytes, size_t nbytes, uint32_t type, size_t rows,
                                size_t cols, size_t n_experts, lt_tensor **out_tensor) {
    if (!ctx || !host_bytes || !out_tensor) return fail(ctx, LT_ERR_INVALID, "null argument");
    *out_tensor = nullptr;
    const size_t be = block_elems(type), bb = block_bytes(type);
    if (!be) return fail(ctx, LT_ERR_UNSUPPORTED, "tensor type %u not supported by the device path", type);
    if (rows == 0 || cols == 0 || n_experts == 0) return fail(ctx, LT_ERR_INVALID, "empty shape");
    if (cols % be) return fail(ctx, LT_ERR_UNSUPPORTED, "cols %zu not a multiple of the %zu-element block", cols, be);
    const size_t total_rows = rows * n_experts;
    const size_t want = total_rows * (cols / be) * bb;
    if (nbytes != want) return fail(ctx, LT_ERR_INVALID, "nbytes %zu != expected %zu", nbytes, want);
    lt_tensor *t = new (std::nothrow) lt_tensor();
    if (!t) return fail(ctx, LT_ERR_OOM, "host allocation failed");
    t->t.type = type;
    t->t.rows = rows;
    t->t.cols = cols;
    t->t.n_experts = n_experts;
    t->t.total_rows = total_rows;
    t->t.bytes = nbytes;
    t->t.blocks_per_row = cols / be;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc((void **)&t->t.base, nbytes);
    if (e != hipSuccess) {
        delete t;
        return hip_fail(ctx, e, "hipMalloc(tensor)");
    }
    set_planes(t->t);
    e = lt::upload_planar(ctx->up, ctx->device, t->t, (const uint8_t *)host_bytes);
    if (e != hipSuccess) {
        (void)hipFree(t->t.base);
        delete t;
        return hip_fail(ctx, e, "tensor upload");
    }
    *out_tensor = t;
    return LT_OK;
}

extern "C" int lt_tensor_read(lt_ctx *ctx, const lt_tensor *t, void *host_bytes, size_t nbytes) {
    if (!ctx || !t || !host_bytes) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (nbytes != t->t.bytes) return fail(ctx, LT_ERR_INVALID, "nbytes %zu != tensor bytes %zu", nbytes, t->t.bytes);
    LT_HIP(ctx, hipSetDevice(ctx->device));
    LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    LT_HIP(ctx, lt::download_planar(ctx->up, t->t, (uint8_t *)host_bytes));
    return LT_OK;
}

extern "C" int lt_tensor_clone(lt_ctx *ctx, const lt_tensor *src, lt_tensor **out_tensor) {
    if (!ctx || !src || !out_tensor) return fail(ctx, LT_ERR_INVALID, "null argument");
    lt_tensor *t = new (std::nothrow) lt_tensor(*src);
    if (!t) return fail(ctx, LT_ERR_OOM, "host allocation failed");
    hipError_t e = hipMalloc((void **)&t->t.base, src->t.bytes);
    if (e == hipSuccess) e = hipMemcpy(t->t.base, src->t.base, src->t.bytes, hipMemcpyDeviceToDevice);
    if (e != hipSuccess) {
        if (t->t.base != src->t.base) (void)hipFree(t->t.base);
        delete t;
        return hip_fail(ctx, e, "tensor clone");
    }
    set_planes(t->t);
    *out_tensor = t;
    return LT_OK;
}

extern "C" int lt_stream_read(lt_ctx *ctx, const void *buf, size_t nbytes) {
    if (!ctx || !buf) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (nbytes == 0 || nbytes % 16 != 0 || ((uintptr_t)buf & 15) != 0)
        return fail(ctx, LT_ERR_INVALID, "nbytes must be a positive multiple of 16 and buf 16-byte aligned");
    int rc = ensure(ctx, ctx->sink, 256);
    if (rc) return rc;
    return launch_rc(ctx, lt::launch_stream_read(buf, nbytes, (uint32_t *)ctx->sink.p, ctx->stream), "stream_read");
}

extern "C" int lt_tensor_free(lt_ctx *ctx, lt_tensor *t) {
    if (!t) return LT_OK;
    if (ctx) (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(t->t.base);
    delete t;
    return LT_OK;
}

extern "C" size_t lt_tensor_bytes(const lt_tensor *t) { return t ? t->t.bytes : 0; }

// ------------------------------------------------------------------ compute
extern "C" int lt_matvec(lt_ctx *ctx, float *out, const lt_tensor *W, const float *x, uint32_t flags) {
    if (!ctx || !out || !x) return fail(ctx, LT_ERR_INVALID, "null argument");
    int rc = check_matvec_tensor(ctx, W);
    if (rc) return rc;
    const DevTensor &T = W->t;
    const bool host = flags & LT_HOST_IO;
    Span span_(ctx, "lt_matvec");
    const float *dx = x;
    float *dy = out;
    if (host) {
        if ((rc = stage_in(ctx, ctx->x, x, T.cols * 4, (const void **)&dx))) return rc;
        if ((rc = ensure(ctx, ctx->out, T.total_rows * 4))) return rc;
        dy = (float *)ctx->out.p;
    } else if (!aligned16(x)) {
        return fail(ctx, LT_ERR_INVALID, "x must be 16-byte aligned");
    }
    if ((rc = matvec_dev(ctx, T, dx, dy))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(out, dy, T.total_rows * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

namespace {

// act(g) * u elementwise, zero tail to n_out (generic dense-FFN path).
__global__ void k_act_mul(const float *g, const float *u, int n, int n_out, uint32_t act, float *h) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = lt::act_apply(act, g[i]) * u[i];
    else if (i < n_out) h[i] = 0.f;
}

// out = Wd * (act(Wg x) * (Wu x)), all device pointers.  Q8_0 weights of a
// shape the single-launch kernel takes run there (unless unfused); others as
// a gate/up launch and a down matvec.
int ffn_dense_dev(lt_ctx *ctx, const DevTensor &G, const DevTensor &U, const DevTensor &D, const float *x,
                  uint32_t act, float *out, bool unfused = false) {
    const size_t F = G.total_rows, Kd = D.cols;
    const bool q8 = G.type == LT_TYPE_Q8_0 && U.type == LT_TYPE_Q8_0 && D.type == LT_TYPE_Q8_0 && Kd == F;
    if (q8 && !unfused) {
        const lt::FfnPlan pl = lt::plan_ffn_fused((int)G.cols, (int)F);
        if (pl.ok) return launch_rc(ctx, lt::launch_ffn_fused(pl, G, U, D, x, act, out, ctx->ffsc, ctx->stream), "ffn_fused");
    }
    int rc = ensure(ctx, ctx->h, Kd * 4);
    if (rc) return rc;
    float *h = (float *)ctx->h.p;
    if (G.type == LT_TYPE_Q8_0 && U.type == LT_TYPE_Q8_0 && Kd == F) {
        if ((rc = launch_rc(ctx, lt::launch_gate_up_q8_0(G, U, x, act, h, ctx->stream), "gate_up_q8_0")))
            return rc;
    } else {
        if ((rc = ensure(ctx, ctx->g, F * 4)) || (rc = ensure(ctx, ctx->u, F * 4))) return rc;
        if ((rc = matvec_dev(ctx, G, x, (float *)ctx->g.p))) return rc;
        if ((rc = matvec_dev(ctx, U, x, (float *)ctx->u.p))) return rc;
        hipLaunchKernelGGL(k_act_mul, dim3((Kd + 255) / 256), dim3(256), 0, ctx->stream, (const float *)ctx->g.p,
                           (const float *)ctx->u.p, (int)F, (int)Kd, act, h);
        if ((rc = launch_rc(ctx, hipGetLastError(), "act_mul"))) return rc;
    }
    return matvec_dev(ctx, D, h, out);
}

int check_ffn(lt_ctx *ctx, const lt_tensor *Wg, const lt_tensor *Wu, const lt_tensor *Wd, size_t d_model) {
    int rc;
    if ((rc = check_matvec_tensor(ctx, Wg)) || (rc = check_matvec_tensor(ctx, Wu)) ||
        (rc = check_matvec_tensor(ctx, Wd)))
        return rc;
    const DevTensor &G = Wg->t, &U = Wu->t, &D = Wd->t;
    if (G.total_rows != U.total_rows || G.cols != U.cols || G.cols != d_model || D.total_rows != d_model ||
        D.cols < G.total_rows)
        return fail(ctx, LT_ERR_INVALID, "dense FFN shapes do not match (gate %zux%zu, up %zux%zu, down %zux%zu)",
                    G.total_rows, G.cols, U.total_rows, U.cols, D.total_rows, D.cols);
    return LT_OK;
}

}  // namespace

extern "C" int lt_ffn_dense(lt_ctx *ctx, float *out, const lt_tensor *Wg, const lt_tensor *Wu,
                            const lt_tensor *Wd, const float *x, uint32_t act, uint32_t flags) {
    if (!ctx || !out || !x || !Wg || !Wu || !Wd) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (act > LT_ACT_GELU_TANH) return fail(ctx, LT_ERR_INVALID, "unknown activation %u", act);
    const size_t D = Wg->t.cols;
    int rc = check_ffn(ctx, Wg, Wu, Wd, D);
    if (rc) return rc;
    Span span_(ctx, "lt_ffn_dense");
    const bool host = flags & LT_HOST_IO;
    const float *dx = x;
    float *dy = out;
    if (host) {
        if ((rc = stage_in(ctx, ctx->x, x, D * 4, (const void **)&dx))) return rc;
        if ((rc = ensure(ctx, ctx->out, D * 4))) return rc;
        dy = (float *)ctx->out.p;
    } else if (!aligned16(x)) {
        return fail(ctx, LT_ERR_INVALID, "x must be 16-byte aligned");
    }
    if ((rc = ffn_dense_dev(ctx, Wg->t, Wu->t, Wd->t, dx, act, dy, (flags & LT_MOE_UNFUSED) != 0))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(out, dy, D * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

namespace {

constexpr uint32_t kMaxK = 16;
constexpr size_t kMaxExperts = 1024;
constexpr size_t kRoutedGateUpMaxExperts = 256;  // top-k inside the gate/up blocks up to here

int check_router(lt_ctx *ctx, const lt_tensor *router, size_t d_model, uint32_t k) {
    if (!router) return fail(ctx, LT_ERR_INVALID, "null router");
    const DevTensor &R = router->t;
    if (R.type != LT_TYPE_F32 && R.type != LT_TYPE_Q8_0)
        return fail(ctx, LT_ERR_UNSUPPORTED, "router type %u (device path: F32, Q8_0)", R.type);
    if (R.cols != d_model) return fail(ctx, LT_ERR_INVALID, "router cols %zu != d_model %zu", R.cols, d_model);
    if (R.total_rows > kMaxExperts) return fail(ctx, LT_ERR_UNSUPPORTED, "more than %zu experts", kMaxExperts);
    if (k == 0 || k > kMaxK || k > R.total_rows)
        return fail(ctx, LT_ERR_INVALID, "k=%u out of range (1..%u, <= n_experts)", k, kMaxK);
    return LT_OK;
}

// logits -> ids/w in context buffers (and scores, if non-NULL); x, bias,
// scores device pointers.
int router_dev(lt_ctx *ctx, const DevTensor &R, const float *x, const float *bias, uint32_t k, uint32_t flags,
               float *scores = nullptr, const lt::RouterPrep *prep = nullptr) {
    int rc;
    if ((rc = ensure(ctx, ctx->logits, R.total_rows * 4)) || (rc = ensure(ctx, ctx->ids, kMaxK * 4)) ||
        (rc = ensure(ctx, ctx->w, kMaxK * 4)))
        return rc;
    float *logits = (float *)ctx->logits.p;
    hipError_t e = lt::launch_router(R, x, bias, logits, ctx->ticket, k, (flags & LT_MOE_NORM_TOPK) ? 1u : 0u,
                                     (uint32_t *)ctx->ids.p, (float *)ctx->w.p, scores, ctx->stream, prep);
    return launch_rc(ctx, e, "router_topk");
}

int stage_bias(lt_ctx *ctx, const float *bias, size_t n, bool host, const float **dbias) {
    *dbias = bias;
    if (bias && host) return stage_in(ctx, ctx->bias, bias, n * 4, (const void **)dbias);
    return LT_OK;
}

int copy_routing_out(lt_ctx *ctx, uint32_t k, uint32_t *ids, float *w, bool host) {
    const hipMemcpyKind kind = host ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    if (ids) LT_HIP(ctx, hipMemcpyAsync(ids, ctx->ids.p, k * 4, kind, ctx->stream));
    if (w) LT_HIP(ctx, hipMemcpyAsync(w, ctx->w.p, k * 4, kind, ctx->stream));
    return LT_OK;
}

// Expert formats: Q4_K (tuned kernels, single-launch layer) and the Gemma4
// APEX formats Q3_K, Q5_0, Q5_1, IQ4_NL (lt_formats.hip).
bool is_fmt(uint32_t t) {
    return t == LT_TYPE_Q5_0 || t == LT_TYPE_Q5_1 || t == LT_TYPE_IQ4_NL || t == LT_TYPE_Q3_K;
}
bool expert_type_ok(uint32_t t) { return t == LT_TYPE_Q4_K || is_fmt(t); }

int check_experts(lt_ctx *ctx, const lt_tensor *gate_up, const lt_tensor *down, size_t d_model, uint32_t d_expert,
                  size_t n_experts, uint32_t k = 0) {
    if (!gate_up || !down) return fail(ctx, LT_ERR_INVALID, "null expert tensor");
    const DevTensor &GU = gate_up->t, &D = down->t;
    if (!expert_type_ok(GU.type) || !expert_type_ok(D.type))
        return fail(ctx, LT_ERR_UNSUPPORTED, "expert types %u/%u (device expert path: Q4_K, Q3_K, Q5_0, Q5_1, IQ4_NL)",
                    GU.type, D.type);
    if (GU.cols != d_model || GU.rows != 2 * (size_t)d_expert)
        return fail(ctx, LT_ERR_INVALID, "gate_up per-expert shape %zux%zu != %ux%zu", GU.rows, GU.cols,
                    2 * d_expert, d_model);
    if (D.rows != d_model || D.cols < d_expert)
        return fail(ctx, LT_ERR_INVALID, "down per-expert shape %zux%zu (need %zu rows, >= %u cols)", D.rows, D.cols,
                    d_model, d_expert);
    if (GU.n_experts != D.n_experts || (n_experts && GU.n_experts != n_experts))
        return fail(ctx, LT_ERR_INVALID, "expert counts differ (gate_up %zu, down %zu, router %zu)", GU.n_experts,
                    D.n_experts, n_experts);
    if (GU.cols > (GU.type == LT_TYPE_Q4_K ? 8192u : 16384u))
        return fail(ctx, LT_ERR_UNSUPPORTED, "d_model %zu too long for the gate/up kernel", GU.cols);
    if (D.type == LT_TYPE_Q4_K && D.blocks_per_row > 16)
        return fail(ctx, LT_ERR_UNSUPPORTED, "down row length %zu > 4096", D.cols);
    if (is_fmt(D.type) && (size_t)(k ? k : 1) * D.cols > 16384)
        return fail(ctx, LT_ERR_UNSUPPORTED, "k * down row length %zu > 16384 (LDS staging of h)",
                    (size_t)(k ? k : 1) * D.cols);
    return LT_OK;
}

// gate/up of the k selected experts into h [k][Kd] (ids on the device)
int gate_up_dev(lt_ctx *ctx, const DevTensor &GU, const float *x, const uint32_t *ids, uint32_t k, uint32_t d_expert,
                uint32_t Kd, uint32_t act, float *h) {
    if (GU.type == LT_TYPE_Q4_K)
        return launch_rc(ctx, lt::launch_expert_gate_up_q4k(GU, x, ids, k, d_expert, Kd, act, h, ctx->stream),
                         "expert_gate_up");
    return launch_rc(ctx, lt::launch_expert_gate_up_fmt(GU, x, ids, k, d_expert, Kd, act, h, ctx->stream),
                     "expert_gate_up_fmt");
}

// gate/up that selects the experts itself from the router logits in
// ctx->logits and leaves the selection in ctx->ids / ctx->w
int gate_up_routed_dev(lt_ctx *ctx, const DevTensor &GU, const float *x, uint32_t k, uint32_t norm,
                       uint32_t d_expert, uint32_t Kd, uint32_t act, float *h) {
    const float *logits = (const float *)ctx->logits.p;
    uint32_t *ids = (uint32_t *)ctx->ids.p;
    float *w = (float *)ctx->w.p;
    if (GU.type == LT_TYPE_Q4_K)
        return launch_rc(ctx,
                         lt::launch_expert_gate_up_q4k_routed(GU, x, logits, k, norm, d_expert, Kd, act, h, ids, w,
                                                              ctx->stream),
                         "expert_gate_up_routed");
    return launch_rc(ctx,
                     lt::launch_expert_gate_up_fmt_routed(GU, x, logits, k, norm, d_expert, Kd, act, h, ids, w,
                                                          ctx->stream),
                     "expert_gate_up_fmt_routed");
}

int down_dev(lt_ctx *ctx, const DevTensor &D, const float *h, const uint32_t *ids, const float *w, uint32_t k,
             const float *base, int accumulate, const float *dscale, float *out) {
    if (D.type == LT_TYPE_Q4_K)
        return launch_rc(ctx, lt::launch_expert_down_q4k(D, h, ids, w, k, base, accumulate, out, ctx->stream, dscale),
                         "expert_down");
    return launch_rc(ctx, lt::launch_expert_down_fmt(D, h, ids, w, k, base, accumulate, dscale, out, ctx->stream),
                     "expert_down_fmt");
}

}  // namespace

extern "C" int lt_moe_router_topk(lt_ctx *ctx, const lt_tensor *router, const float *x, const float *bias,
                                  uint32_t k, uint32_t flags, uint32_t *ids, float *weights, float *scores) {
    if (!ctx || !x || !router || !ids || !weights) return fail(ctx, LT_ERR_INVALID, "null argument");
    int rc = check_router(ctx, router, router->t.cols, k);
    if (rc) return rc;
    const DevTensor &R = router->t;
    const bool host = flags & LT_HOST_IO;
    const float *dx = x, *dbias = bias;
    Span span_(ctx, "lt_moe_router_topk");
    float *dscores = scores;
    if (host) {
        if ((rc = stage_in(ctx, ctx->x, x, R.cols * 4, (const void **)&dx))) return rc;
        if (scores) {
            if ((rc = ensure(ctx, ctx->out, R.total_rows * 4))) return rc;
            dscores = (float *)ctx->out.p;
        }
    }
    if ((rc = stage_bias(ctx, bias, R.total_rows, host, &dbias))) return rc;
    if ((rc = router_dev(ctx, R, dx, dbias, k, flags, dscores))) return rc;
    if ((rc = copy_routing_out(ctx, k, ids, weights, host))) return rc;
    if (host) {
        if (scores)
            LT_HIP(ctx, hipMemcpyAsync(scores, dscores, R.total_rows * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

extern "C" int lt_expert_gate_up_id(lt_ctx *ctx, const lt_tensor *gate_up, const float *x, const uint32_t *ids,
                                    uint32_t k, uint32_t d_expert, uint32_t down_cols, uint32_t act, float *h,
                                    uint32_t flags) {
    if (!ctx || !gate_up || !x || !ids || !h) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (k == 0 || k > kMaxK) return fail(ctx, LT_ERR_INVALID, "k=%u out of range", k);
    if (act > LT_ACT_GELU_TANH) return fail(ctx, LT_ERR_INVALID, "unknown activation %u", act);
    const DevTensor &GU = gate_up->t;
    if (!expert_type_ok(GU.type)) return fail(ctx, LT_ERR_UNSUPPORTED, "gate_up type %u not on the device path", GU.type);
    if (GU.rows != 2 * (size_t)d_expert) return fail(ctx, LT_ERR_INVALID, "gate_up rows %zu != 2*d_expert", GU.rows);
    if (down_cols < d_expert || down_cols % (GU.type == LT_TYPE_Q4_K ? 256 : 32))
        return fail(ctx, LT_ERR_INVALID, "down_cols %u", down_cols);
    if (GU.cols > (GU.type == LT_TYPE_Q4_K ? 8192u : 16384u))
        return fail(ctx, LT_ERR_UNSUPPORTED, "d_model %zu too long for the gate/up kernel", GU.cols);
    const bool host = flags & LT_HOST_IO;
    const float *dx = x;
    const uint32_t *dids = ids;
    float *dh = h;
    Span span_(ctx, "lt_expert_gate_up_id");
    int rc;
    if (host) {
        for (uint32_t s = 0; s < k; s++)
            if (ids[s] >= GU.n_experts) return fail(ctx, LT_ERR_INVALID, "ids[%u]=%u >= n_experts", s, ids[s]);
        if ((rc = stage_in(ctx, ctx->x, x, GU.cols * 4, (const void **)&dx))) return rc;
        if ((rc = stage_in(ctx, ctx->ids_io, ids, k * 4, (const void **)&dids))) return rc;
        if ((rc = ensure(ctx, ctx->out, (size_t)k * down_cols * 4))) return rc;
        dh = (float *)ctx->out.p;
    } else if (!aligned16(x)) {
        return fail(ctx, LT_ERR_INVALID, "x must be 16-byte aligned");
    }
    if ((rc = gate_up_dev(ctx, GU, dx, dids, k, d_expert, down_cols, act, dh))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(h, dh, (size_t)k * down_cols * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

extern "C" int lt_expert_down_id(lt_ctx *ctx, const lt_tensor *down, const float *h, const uint32_t *ids,
                                 const float *weights, uint32_t k, float *out, uint32_t flags) {
    if (!ctx || !down || !h || !ids || !weights || !out) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (k == 0 || k > kMaxK) return fail(ctx, LT_ERR_INVALID, "k=%u out of range", k);
    const DevTensor &D = down->t;
    if (!expert_type_ok(D.type)) return fail(ctx, LT_ERR_UNSUPPORTED, "down type %u not on the device path", D.type);
    if (D.type == LT_TYPE_Q4_K && D.blocks_per_row > 16)
        return fail(ctx, LT_ERR_UNSUPPORTED, "down row length %zu > 4096", D.cols);
    if (is_fmt(D.type) && (size_t)k * D.cols > 16384)
        return fail(ctx, LT_ERR_UNSUPPORTED, "k * down row length > 16384 (LDS staging of h)");
    const bool host = flags & LT_HOST_IO;
    const float *dh = h, *dw = weights;
    Span span_(ctx, "lt_expert_down_id");
    const uint32_t *dids = ids;
    float *dout = out;
    int rc;
    if (host) {
        for (uint32_t s = 0; s < k; s++)
            if (ids[s] >= D.n_experts) return fail(ctx, LT_ERR_INVALID, "ids[%u]=%u >= n_experts", s, ids[s]);
        if ((rc = stage_in(ctx, ctx->h, h, (size_t)k * D.cols * 4, (const void **)&dh))) return rc;
        if ((rc = stage_in(ctx, ctx->ids_io, ids, k * 4, (const void **)&dids))) return rc;
        if ((rc = stage_in(ctx, ctx->w_io, weights, k * 4, (const void **)&dw))) return rc;
        if (flags & LT_MOE_ACCUMULATE) {
            if ((rc = stage_in(ctx, ctx->out, out, D.rows * 4, (const void **)&dout))) return rc;
        } else if ((rc = ensure(ctx, ctx->out, D.rows * 4))) {
            return rc;
        }
        dout = (float *)ctx->out.p;
    } else if (!aligned16(h)) {
        return fail(ctx, LT_ERR_INVALID, "h must be 16-byte aligned");
    }
    if ((rc = down_dev(ctx, D, dh, dids, dw, k, nullptr, (flags & LT_MOE_ACCUMULATE) ? 1 : 0, nullptr, dout)))
        return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(out, dout, D.rows * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

namespace {

// A Q8_0 dense FFN the fused kernel computes itself: gate and up [S][D],
// down [D][S] (no padding of the down rows), 256 <= S <= 4096.
bool shared_fusable(const DevTensor &G, const DevTensor &U, const DevTensor &Dn) {
    return G.type == LT_TYPE_Q8_0 && U.type == LT_TYPE_Q8_0 && Dn.type == LT_TYPE_Q8_0 &&
           Dn.cols == G.total_rows && G.total_rows >= 256 && G.total_rows <= (size_t)lt::kFusedMaxShared;
}

// The fused kernel's description of a layer (sg null: no shared FFN; R, GU,
// Dn null and k 0: the dense FFN alone).
lt::FusedLayer fused_layer(const DevTensor &R, const DevTensor &GU, const DevTensor &Dn, const lt_tensor *sg,
                           const lt_tensor *su, const lt_tensor *sd, uint32_t k, uint32_t d_expert, uint32_t flags) {
    lt::FusedLayer L{};
    L.det = (flags & LT_MOE_DETERMINISTIC) ? 1 : 0;
    L.R = &R;
    L.GU = &GU;
    L.Dn = &Dn;
    L.E = (int)R.total_rows;
    L.D = (int)GU.cols;
    L.F = (int)d_expert;
    L.Kd = (int)Dn.cols;
    L.k = (int)k;
    if (sg) {
        L.SG = &sg->t;
        L.SU = &su->t;
        L.SD = &sd->t;
        L.S = (int)sg->t.total_rows;
    }
    return L;
}

// The decode MoE layer on device pointers.
int moe_dev(lt_ctx *ctx, float *out, const float *x, const DevTensor &R, const float *bias, const DevTensor &GU,
            const DevTensor &D, const lt_tensor *sh_gate, const lt_tensor *sh_up, const lt_tensor *sh_down,
            uint32_t k, uint32_t d_expert, uint32_t act, uint32_t flags) {
    int rc;
    const size_t Kd = D.cols;
    // (Q4_K experts, or the APEX formats: Q3_K gate/up, IQ4_NL / Q5_0 / Q5_1
    // down; the plan checks the shapes)
    const bool fusable = !(flags & LT_MOE_UNFUSED) && (R.type == LT_TYPE_F32 || R.type == LT_TYPE_Q8_0) &&
                         (GU.type == LT_TYPE_Q4_K || GU.type == LT_TYPE_Q3_K) &&
                         (D.type == LT_TYPE_Q4_K || D.type == LT_TYPE_IQ4_NL || D.type == LT_TYPE_Q5_0 ||
                          D.type == LT_TYPE_Q5_1);
    // the shared FFN inside the same launch: Q8_0, unpadded down, atomic combine
    bool sh_in = fusable && sh_gate && shared_fusable(sh_gate->t, sh_up->t, sh_down->t) &&
                 !(flags & LT_MOE_DETERMINISTIC);
    if (fusable) {
        lt::FusedPlan pl = lt::plan_moe_fused(fused_layer(R, GU, D, sh_in ? sh_gate : nullptr, sh_up, sh_down, k,
                                                          d_expert, flags));
        if (!pl.ok && sh_in) {  // no room for the shared FFN's blocks: it runs first, as the base
            sh_in = false;
            pl = lt::plan_moe_fused(fused_layer(R, GU, D, nullptr, nullptr, nullptr, k, d_expert, flags));
        }
        if (pl.ok) {
            const float *base = nullptr;
            if (sh_gate && !sh_in) {
                if ((rc = ensure(ctx, ctx->shared, D.rows * 4))) return rc;
                if ((rc = ffn_dense_dev(ctx, sh_gate->t, sh_up->t, sh_down->t, x, act, (float *)ctx->shared.p)))
                    return rc;
                base = (const float *)ctx->shared.p;
            }
            if ((rc = ensure_fused(ctx)) || (rc = ensure(ctx, ctx->ids, kMaxK * 4)) ||
                (rc = ensure(ctx, ctx->w, kMaxK * 4)))
                return rc;
            ctx->prof.stamps_pending = ctx->prof.stamps != nullptr;
            return launch_rc(ctx,
                             lt::launch_moe_fused(pl,
                                                  fused_layer(R, GU, D, sh_in ? sh_gate : nullptr, sh_up, sh_down,
                                                              k, d_expert, flags),
                                                  bias, x, act, (flags & LT_MOE_NORM_TOPK) ? 1u : 0u, base,
                                                  (flags & LT_MOE_ACCUMULATE) ? 1 : 0,
                                                  (flags & LT_MOE_DETERMINISTIC) ? 1 : 0, out, (uint32_t *)ctx->ids.p,
                                                  (float *)ctx->w.p, ctx->fsc, ctx->stream),
                             "moe_fused");
        }
    }
    const float *base = nullptr;
    if (sh_gate) {
        if ((rc = ensure(ctx, ctx->shared, D.rows * 4))) return rc;
        if ((rc = ffn_dense_dev(ctx, sh_gate->t, sh_up->t, sh_down->t, x, act, (float *)ctx->shared.p,
                                (flags & LT_MOE_UNFUSED) != 0)))
            return rc;
        base = (const float *)ctx->shared.p;
    }
    if ((rc = ensure(ctx, ctx->eh, (size_t)k * Kd * 4))) return rc;
    float *h = (float *)ctx->eh.p;
    if (R.total_rows <= kRoutedGateUpMaxExperts) {
        // logits only; each gate/up block selects its expert from them
        if ((rc = router_dev(ctx, R, x, bias, 0, flags))) return rc;
        rc = gate_up_routed_dev(ctx, GU, x, k, (flags & LT_MOE_NORM_TOPK) ? 1u : 0u, d_expert, (uint32_t)Kd, act, h);
    } else {
        if ((rc = router_dev(ctx, R, x, bias, k, flags))) return rc;
        rc = gate_up_dev(ctx, GU, x, (const uint32_t *)ctx->ids.p, k, d_expert, (uint32_t)Kd, act, h);
    }
    if (rc) return rc;
    return down_dev(ctx, D, h, (const uint32_t *)ctx->ids.p, (const float *)ctx->w.p, k, base,
                    (flags & LT_MOE_ACCUMULATE) ? 1 : 0, nullptr, out);
}

}  // namespace

extern "C" int lt_moe_forward(lt_ctx *ctx, float *out, const float *x, const lt_tensor *router,
                              const float *router_bias, const lt_tensor *gate_up, const lt_tensor *down,
                              const lt_tensor *sh_gate, const lt_tensor *sh_up, const lt_tensor *sh_down, uint32_t k,
                              uint32_t d_expert, uint32_t act, uint32_t flags, uint32_t *out_ids, float *out_w) {
    if (!ctx || !out || !x) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (act > LT_ACT_GELU_TANH) return fail(ctx, LT_ERR_INVALID, "unknown activation %u", act);
    if (!router || !gate_up || !down) return fail(ctx, LT_ERR_INVALID, "null tensor");
    const size_t d_model = gate_up->t.cols;
    int rc;
    if ((rc = check_router(ctx, router, d_model, k))) return rc;
    if ((rc = check_experts(ctx, gate_up, down, d_model, d_expert, router->t.total_rows, k))) return rc;
    const bool shared = sh_gate || sh_up || sh_down;
    if (shared) {
        if (!sh_gate || !sh_up || !sh_down) return fail(ctx, LT_ERR_INVALID, "shared FFN needs gate, up and down");
        if ((rc = check_ffn(ctx, sh_gate, sh_up, sh_down, d_model))) return rc;
    }
    Span span_(ctx, "lt_moe_forward");
    const bool host = flags & LT_HOST_IO;
    const float *dx = x, *dbias = router_bias;
    float *dout = out;
    if (host) {
        if ((rc = stage_in(ctx, ctx->x, x, d_model * 4, (const void **)&dx))) return rc;
        if (flags & LT_MOE_ACCUMULATE) {
            if ((rc = stage_in(ctx, ctx->out, out, d_model * 4, (const void **)&dout))) return rc;
        } else if ((rc = ensure(ctx, ctx->out, d_model * 4))) {
            return rc;
        }
        dout = (float *)ctx->out.p;
    } else if (!aligned16(x)) {
        return fail(ctx, LT_ERR_INVALID, "x must be 16-byte aligned");
    }
    if ((rc = stage_bias(ctx, router_bias, router->t.total_rows, host, &dbias))) return rc;
    rc = moe_dev(ctx, dout, dx, router->t, dbias, gate_up->t, down->t, shared ? sh_gate : nullptr, sh_up, sh_down, k,
                 d_expert, act, flags);
    if (rc) return rc;
    if ((rc = copy_routing_out(ctx, k, out_ids, out_w, host))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(out, dout, d_model * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
        return check_fused_err(ctx);
    }
    return LT_OK;
}

extern "C" int lt_moe_forward_noalloc(lt_ctx *ctx, float *out, const float *x, const lt_tensor *router,
                                      const float *router_bias, const lt_tensor *gate_up, const lt_tensor *down,
                                      const lt_tensor *sh_gate, const lt_tensor *sh_up, const lt_tensor *sh_down,
                                      uint32_t k, uint32_t d_expert, uint32_t act, uint32_t flags, uint32_t *out_ids,
                                      float *out_w) {
    if (!ctx || !out || !x) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (act > LT_ACT_GELU_TANH) return fail(ctx, LT_ERR_INVALID, "unknown activation %u", act);
    if (!router || !gate_up || !down) return fail(ctx, LT_ERR_INVALID, "null tensor");
    if (flags & ~(uint32_t)(LT_MOE_NORM_TOPK | LT_MOE_ACCUMULATE | LT_MOE_DETERMINISTIC))
        return fail(ctx, LT_ERR_INVALID,
                    "allocation-free MoE: flags 0x%x not allowed (device pointers only: no LT_HOST_IO; no "
                    "LT_MOE_UNFUSED)",
                    flags & ~(uint32_t)(LT_MOE_NORM_TOPK | LT_MOE_ACCUMULATE | LT_MOE_DETERMINISTIC));
    const size_t d_model = gate_up->t.cols;
    int rc;
    if ((rc = check_router(ctx, router, d_model, k))) return rc;
    if ((rc = check_experts(ctx, gate_up, down, d_model, d_expert, router->t.total_rows, k))) return rc;
    const bool shared = sh_gate || sh_up || sh_down;
    if (shared) {
        if (!sh_gate || !sh_up || !sh_down) return fail(ctx, LT_ERR_INVALID, "shared FFN needs gate, up and down");
        if ((rc = check_ffn(ctx, sh_gate, sh_up, sh_down, d_model))) return rc;
        if (!shared_fusable(sh_gate->t, sh_up->t, sh_down->t) || (flags & LT_MOE_DETERMINISTIC))
            return fail(ctx, LT_ERR_UNSUPPORTED,
                        "allocation-free MoE: a shared FFN must be Q8_0 with down K == d_ffn in 256..%d, and "
                        "the combine atomic (no LT_MOE_DETERMINISTIC)",
                        lt::kFusedMaxShared);
    }
    if (!aligned16(x)) return fail(ctx, LT_ERR_INVALID, "x must be 16-byte aligned");
    const DevTensor &R = router->t, &GU = gate_up->t, &D = down->t;
    if ((R.type != LT_TYPE_F32 && R.type != LT_TYPE_Q8_0) || GU.type != LT_TYPE_Q4_K || D.type != LT_TYPE_Q4_K)
        return fail(ctx, LT_ERR_UNSUPPORTED,
                    "allocation-free MoE: single-launch kernel only (F32 or Q8_0 router, Q4_K gate_up and down)");
    const lt::FusedLayer L = fused_layer(R, GU, D, shared ? sh_gate : nullptr, sh_up, sh_down, k, d_expert, flags);
    const lt::FusedPlan pl = lt::plan_moe_fused(L);
    if (!pl.ok)
        return fail(ctx, LT_ERR_UNSUPPORTED,
                    "allocation-free MoE: shape beyond the static scratch's kernel (d_model %zu, %zu experts, "
                    "d_expert %u, down K %zu, k %u%s; limits: d_model 256..4096 in steps of 256, down K <= 1024, "
                    "<= 256 experts, k <= 16, and the grid's room for the shared FFN)",
                    GU.cols, R.total_rows, d_expert, D.cols, k, shared ? ", shared FFN" : "");
    ctx->prof.stamps_pending = ctx->prof.stamps != nullptr;
    uint32_t *ids_dev = (uint32_t *)(ctx->na_base + lt::kFusedIdsOff);
    float *w_dev = (float *)(ctx->na_base + lt::kFusedWOff);
    rc = launch_rc(ctx,
                   lt::launch_moe_fused(pl, L, router_bias, x, act, (flags & LT_MOE_NORM_TOPK) ? 1u : 0u, nullptr,
                                        (flags & LT_MOE_ACCUMULATE) ? 1 : 0, (flags & LT_MOE_DETERMINISTIC) ? 1 : 0,
                                        out, ids_dev, w_dev, ctx->na_fsc, ctx->stream),
                   "moe_fused (allocation-free)");
    if (rc) return rc;
    if (out_ids) LT_HIP(ctx, hipMemcpyAsync(out_ids, ids_dev, k * 4, hipMemcpyDeviceToDevice, ctx->stream));
    if (out_w) LT_HIP(ctx, hipMemcpyAsync(out_w, w_dev, k * 4, hipMemcpyDeviceToDevice, ctx->stream));
    return LT_OK;
}

extern "C" int lt_moe_prefill(lt_ctx *ctx, float *out, const float *X, uint32_t T, const lt_tensor *router,
                              const float *router_bias, const lt_tensor *gate_up, const lt_tensor *down, uint32_t k,
                              uint32_t d_expert, uint32_t act, uint32_t flags, uint32_t *out_ids, float *out_w) {
    if (!ctx || !out || !X) return fail(ctx, LT_ERR_INVALID, "null argument");
    if (T == 0 || T > 65536) return fail(ctx, LT_ERR_INVALID, "T=%u out of range (1..65536)", T);
    if (act > LT_ACT_GELU_TANH) return fail(ctx, LT_ERR_INVALID, "unknown activation %u", act);
    if (!router || !gate_up || !down) return fail(ctx, LT_ERR_INVALID, "null tensor");
    if (flags & LT_MOE_ACCUMULATE) return fail(ctx, LT_ERR_UNSUPPORTED, "prefill does not accumulate");
    const size_t D = gate_up->t.cols;
    int rc;
    if ((rc = check_router(ctx, router, D, k))) return rc;
    if ((rc = check_experts(ctx, gate_up, down, D, d_expert, router->t.total_rows))) return rc;
    if (gate_up->t.type != LT_TYPE_Q4_K || down->t.type != LT_TYPE_Q4_K)
        return fail(ctx, LT_ERR_UNSUPPORTED, "batched prefill takes Q4_K experts");
    if (d_expert % 64 || D % 128)
        return fail(ctx, LT_ERR_UNSUPPORTED, "prefill tiles need d_expert %% 64 == 0 and d_model %% 128 == 0");
    if ((size_t)T * k > (1u << 20)) return fail(ctx, LT_ERR_UNSUPPORTED, "T*k > 2^20");
    const int E = (int)router->t.total_rows, Kd = (int)down->t.cols;
    Span span_(ctx, "lt_moe_prefill");
    const bool host = flags & LT_HOST_IO;
    const float *dX = X, *dbias = router_bias;
    float *dout = out;
    uint32_t *dids = out_ids;
    float *dw = out_w;
    if (host) {
        if ((rc = stage_in(ctx, ctx->x, X, (size_t)T * D * 4, (const void **)&dX))) return rc;
        if ((rc = ensure(ctx, ctx->out, (size_t)T * D * 4))) return rc;
        dout = (float *)ctx->out.p;
        dids = nullptr;  // copied from the workspace below
        dw = nullptr;
    } else if (!aligned16(X) || !aligned16(out)) {
        return fail(ctx, LT_ERR_INVALID, "X and out must be 16-byte aligned");
    }
    if ((rc = stage_bias(ctx, router_bias, E, host, &dbias))) return rc;
    const size_t wsb = lt::prefill_workspace_bytes((int)T, (int)k, E, Kd, (int)D);
    if ((rc = ensure(ctx, ctx->pf, wsb))) return rc;
    rc = launch_rc(ctx,
                   lt::launch_moe_prefill(router->t, gate_up->t, down->t, dX, (int)T, dbias, (int)k, (int)d_expert,
                                          act, (flags & LT_MOE_NORM_TOPK) ? 1u : 0u, ctx->pf.p, dout, dids, dw,
                                          ctx->err_dev, ctx->xcd_local, ctx->stream),
                   "moe_prefill");
    if (rc) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(out, dout, (size_t)T * D * 4, hipMemcpyDeviceToHost, ctx->stream));
        // ids and weights sit right after the logits in the workspace
        const size_t logits_b = ((size_t)T * E * 4 + 255) & ~(size_t)255;
        const size_t ids_b = ((size_t)T * k * 4 + 255) & ~(size_t)255;
        const uint8_t *wsp = (const uint8_t *)ctx->pf.p;
        if (out_ids)
            LT_HIP(ctx, hipMemcpyAsync(out_ids, wsp + logits_b, (size_t)T * k * 4, hipMemcpyDeviceToHost, ctx->stream));
        if (out_w)
            LT_HIP(ctx, hipMemcpyAsync(out_w, wsp + logits_b + ids_b, (size_t)T * k * 4, hipMemcpyDeviceToHost,
                                       ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
        return check_fused_err(ctx);
    }
    return LT_OK;
}

// ------------------------------------------------------------- norms, Gemma4 block
namespace {

constexpr uint32_t kNormFlags = LT_HOST_IO | LT_NORM_PRECISE | LT_NORM_ONE_PLUS_W;

// 256-byte aligned float slices of ctx->nrm, sized up front by need().
struct Arena {
    size_t bytes = 0;
    uint8_t *base = nullptr;
    static size_t round(size_t n) { return (n * 4 + 255) & ~(size_t)255; }
    void need(size_t n) { bytes += round(n); }
    float *take(size_t n) {
        float *p = reinterpret_cast<float *>(base);
        base += round(n);
        return p;
    }
};

int arena_open(lt_ctx *ctx, Arena &a) {
    int rc = ensure(ctx, ctx->nrm, a.bytes);
    if (rc) return rc;
    a.base = (uint8_t *)ctx->nrm.p;
    return LT_OK;
}

// Host input -> arena slice (LT_HOST_IO), or the device pointer itself.
int io_in(lt_ctx *ctx, bool host, Arena &a, const float *src, size_t n, const float **dst) {
    if (!src || !host) {
        *dst = src;
        return LT_OK;
    }
    float *d = a.take(n);
    LT_HIP(ctx, hipMemcpyAsync(d, src, n * 4, hipMemcpyHostToDevice, ctx->stream));
    *dst = d;
    return LT_OK;
}

int check_norm(lt_ctx *ctx, uint32_t rows, uint32_t n, float eps, uint32_t flags, uint32_t allowed) {
    if (n == 0 || n > (uint32_t)lt::kMaxNormCols)
        return fail(ctx, LT_ERR_UNSUPPORTED, "row length %u (device norms: 1..%d)", n, lt::kMaxNormCols);
    if (rows == 0 || rows > 65536) return fail(ctx, LT_ERR_INVALID, "rows=%u out of range (1..65536)", rows);
    if (!(eps >= 0.0f) || eps > 1.0f) return fail(ctx, LT_ERR_INVALID, "eps must be in [0, 1]");
    if (flags & ~allowed) return fail(ctx, LT_ERR_INVALID, "unknown flags 0x%x", flags & ~allowed);
    return LT_OK;
}

int norm_run(lt_ctx *ctx, int op, const float *a, const float *b, const float *w, const float *w2, float *out,
             float *out2, uint32_t rows, uint32_t n, float eps, float scale, uint32_t flags) {
    return launch_rc(ctx,
                     lt::launch_norm(op, a, b, w, w2, out, out2, (int)rows, (int)n, eps, scale,
                                     (flags & LT_NORM_PRECISE) ? 1 : 0, (flags & LT_NORM_ONE_PLUS_W) ? 1 : 0,
                                     ctx->stream),
                     "rmsnorm");
}

// Shared body of lt_rmsnorm / lt_add_rmsnorm.
int rmsnorm_entry(lt_ctx *ctx, int op, float *out, const float *a, const float *b, const float *w, uint32_t rows,
                  uint32_t n, float eps, uint32_t flags) {
    int rc = check_norm(ctx, rows, n, eps, flags, kNormFlags);
    if (rc) return rc;
    Span span_(ctx, op ? "lt_add_rmsnorm" : "lt_rmsnorm");
    const bool host = flags & LT_HOST_IO;
    const size_t len = (size_t)rows * n;
    Arena ar;
    if (host) {
        ar.need(len), ar.need(len), ar.need(n);
        if (b) ar.need(len);
        if ((rc = arena_open(ctx, ar))) return rc;
    }
    const float *da, *db, *dw;
    if ((rc = io_in(ctx, host, ar, a, len, &da)) || (rc = io_in(ctx, host, ar, b, len, &db)) ||
        (rc = io_in(ctx, host, ar, w, n, &dw)))
        return rc;
    float *dout = host ? ar.take(len) : out;
    if ((rc = norm_run(ctx, op, da, db, dw, nullptr, dout, nullptr, rows, n, eps, 1.0f, flags))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(out, dout, len * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

}  // namespace

extern "C" int lt_rmsnorm(lt_ctx *ctx, float *out, const float *x, const float *w, uint32_t rows, uint32_t n,
                          float eps, uint32_t flags) {
    if (!ctx || !out || !x) return fail(ctx, LT_ERR_INVALID, "null argument");
    return rmsnorm_entry(ctx, 0, out, x, nullptr, w, rows, n, eps, flags);
}

extern "C" int lt_add_rmsnorm(lt_ctx *ctx, float *out, const float *a, const float *b, const float *w, uint32_t rows,
                              uint32_t n, float eps, uint32_t flags) {
    if (!ctx || !out || !a || !b || !w) return fail(ctx, LT_ERR_INVALID, "null argument");
    return rmsnorm_entry(ctx, 1, out, a, b, w, rows, n, eps, flags);
}

extern "C" int lt_rmsnorm_weighted_raw_scaled(lt_ctx *ctx, float *weighted_out, float *raw_scaled_out,
                                              const float *x, const float *w, const float *raw_scale,
                                              float raw_global_scale, uint32_t n, float eps, uint32_t flags) {
    if (!ctx || !weighted_out || !raw_scaled_out || !x || !w || !raw_scale)
        return fail(ctx, LT_ERR_INVALID, "null argument");
    int rc = check_norm(ctx, 1, n, eps, flags, LT_HOST_IO | LT_NORM_PRECISE);
    if (rc) return rc;
    Span span_(ctx, "lt_rmsnorm_weighted_raw_scaled");
    const bool host = flags & LT_HOST_IO;
    Arena ar;
    if (host) {
        for (int i = 0; i < 5; i++) ar.need(n);
        if ((rc = arena_open(ctx, ar))) return rc;
    }
    const float *dx, *dw, *ds;
    if ((rc = io_in(ctx, host, ar, x, n, &dx)) || (rc = io_in(ctx, host, ar, w, n, &dw)) ||
        (rc = io_in(ctx, host, ar, raw_scale, n, &ds)))
        return rc;
    float *dwo = host ? ar.take(n) : weighted_out, *dro = host ? ar.take(n) : raw_scaled_out;
    if ((rc = norm_run(ctx, 2, dx, nullptr, dw, ds, dwo, dro, 1, n, eps, raw_global_scale, flags))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(weighted_out, dwo, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipMemcpyAsync(raw_scaled_out, dro, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

extern "C" int lt_moe_tail(lt_ctx *ctx, float *x, const float *moe, const float *dense_ffn,
                           const float *post_ffw_norm_2, const float *post_ffw_norm, float layer_output_scale,
                           uint32_t n, float eps, uint32_t flags) {
    if (!ctx || !x || !moe || !dense_ffn || !post_ffw_norm_2 || !post_ffw_norm)
        return fail(ctx, LT_ERR_INVALID, "null argument");
    int rc = check_norm(ctx, 1, n, eps, flags, LT_HOST_IO | LT_NORM_PRECISE);
    if (rc) return rc;
    Span span_(ctx, "lt_moe_tail");
    const bool host = flags & LT_HOST_IO;
    Arena ar;
    if (host) {
        for (int i = 0; i < 5; i++) ar.need(n);
        if ((rc = arena_open(ctx, ar))) return rc;
    }
    const float *dm, *dd, *dw2, *dw, *dx;
    if ((rc = io_in(ctx, host, ar, moe, n, &dm)) || (rc = io_in(ctx, host, ar, dense_ffn, n, &dd)) ||
        (rc = io_in(ctx, host, ar, post_ffw_norm_2, n, &dw2)) || (rc = io_in(ctx, host, ar, post_ffw_norm, n, &dw)) ||
        (rc = io_in(ctx, host, ar, x, n, &dx)))
        return rc;
    float *xo = const_cast<float *>(dx);
    if ((rc = norm_run(ctx, 3, dm, dd, dw, dw2, xo, nullptr, 1, n, eps, layer_output_scale, flags))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(x, xo, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

extern "C" int lt_gemma4_moe_block(lt_ctx *ctx, float *x, const float *dense_ffn, const lt_tensor *router,
                                   const lt_tensor *gate_up, const lt_tensor *down, const float *pre_ffw_norm_2,
                                   const float *router_scale, const float *down_exps_scale,
                                   const float *post_ffw_norm_2, const float *post_ffw_norm,
                                   float layer_output_scale, float eps, uint32_t k, uint32_t d_expert, uint32_t act,
                                   uint32_t flags, uint32_t *out_ids, float *out_w) {
    if (!ctx || !x || !dense_ffn || !pre_ffw_norm_2 || !router_scale || !post_ffw_norm_2 || !post_ffw_norm)
        return fail(ctx, LT_ERR_INVALID, "null argument");
    if (act > LT_ACT_GELU_TANH) return fail(ctx, LT_ERR_INVALID, "unknown activation %u", act);
    if (!router || !gate_up || !down) return fail(ctx, LT_ERR_INVALID, "null tensor");
    const size_t n = gate_up->t.cols;
    int rc;
    if ((rc = check_router(ctx, router, n, k))) return rc;
    if ((rc = check_experts(ctx, gate_up, down, n, d_expert, router->t.total_rows, k))) return rc;
    if ((rc = check_norm(ctx, 1, (uint32_t)n, eps, flags,
                         LT_HOST_IO | LT_NORM_PRECISE | LT_MOE_NORM_TOPK | LT_MOE_UNFUSED | LT_MOE_DETERMINISTIC)))
        return rc;
    const DevTensor &R = router->t, &GU = gate_up->t, &D = down->t;
    const size_t E = R.total_rows, Kd = D.cols;
    Span span_(ctx, "lt_gemma4_moe_block");
    const bool host = flags & LT_HOST_IO;
    if (!host && !aligned16(x)) return fail(ctx, LT_ERR_INVALID, "x must be 16-byte aligned");
    Arena ar;
    for (int i = 0; i < 3; i++) ar.need(n);  // moe_in, router_in, moe
    if (host) {
        for (int i = 0; i < 6; i++) ar.need(n);  // x, dense, four norm vectors
        ar.need(E);
    }
    if ((rc = arena_open(ctx, ar))) return rc;
    float *moe_in = ar.take(n), *router_in = ar.take(n), *moe = ar.take(n);
    const float *dx, *dd, *dpre, *drs, *dds, *dp2, *dp;
    if ((rc = io_in(ctx, host, ar, x, n, &dx)) || (rc = io_in(ctx, host, ar, dense_ffn, n, &dd)) ||
        (rc = io_in(ctx, host, ar, pre_ffw_norm_2, n, &dpre)) || (rc = io_in(ctx, host, ar, router_scale, n, &drs)) ||
        (rc = io_in(ctx, host, ar, down_exps_scale, E, &dds)) ||
        (rc = io_in(ctx, host, ar, post_ffw_norm_2, n, &dp2)) || (rc = io_in(ctx, host, ar, post_ffw_norm, n, &dp)))
        return rc;
    float *xio = const_cast<float *>(dx);
    const float inv_sqrt_d = 1.0f / sqrtf((float)n);
    // the whole block in one launch of the single-launch MoE kernel: Q8_0
    // router, Q4_K or APEX experts, the tree order of the norms (LT_NORM_PRECISE
    // keeps the reference's sequential sums, LT_MOE_DETERMINISTIC the slot
    // order of the experts' adds: the launches below)
    if (!(flags & (LT_NORM_PRECISE | LT_MOE_UNFUSED | LT_MOE_DETERMINISTIC)) && R.type == LT_TYPE_Q8_0 &&
        (GU.type == LT_TYPE_Q4_K || GU.type == LT_TYPE_Q3_K) &&
        (D.type == LT_TYPE_Q4_K || D.type == LT_TYPE_IQ4_NL || D.type == LT_TYPE_Q5_0 || D.type == LT_TYPE_Q5_1)) {
        const lt::GemmaBlock gb{drs, dpre, dds, dd, dp2, dp, xio, inv_sqrt_d, eps, layer_output_scale};
        lt::FusedLayer L = fused_layer(R, GU, D, nullptr, nullptr, nullptr, k, d_expert, flags);
        L.gb = &gb;
        const lt::FusedPlan pl = lt::plan_moe_fused(L);
        if (pl.ok && pl.gemma) {
            if ((rc = ensure_fused(ctx)) || (rc = ensure(ctx, ctx->ids, kMaxK * 4)) ||
                (rc = ensure(ctx, ctx->w, kMaxK * 4)))
                return rc;
            ctx->prof.stamps_pending = ctx->prof.stamps != nullptr;
            rc = launch_rc(ctx,
                           lt::launch_moe_fused(pl, L, nullptr, dx, act, (flags & LT_MOE_NORM_TOPK) ? 1u : 0u, nullptr,
                                                0, 0, moe, (uint32_t *)ctx->ids.p, (float *)ctx->w.p, ctx->fsc,
                                                ctx->stream),
                           "gemma4_block_fused");
            if (rc) return rc;
            if ((rc = copy_routing_out(ctx, k, out_ids, out_w, host))) return rc;
            if (host) {
                LT_HIP(ctx, hipMemcpyAsync(x, xio, n * 4, hipMemcpyDeviceToHost, ctx->stream));
                LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
                prof_harvest(ctx);
                return check_fused_err(ctx);
            }
            return LT_OK;
        }
    }
    // gemma4/forward.zig:405-414: expert input and router input from one RMS
    // of x -- inside the Q8_0 router with the tree sum, else a kernel of its own
    const bool fuse_prep = !(flags & LT_NORM_PRECISE) && R.type == LT_TYPE_Q8_0;
    const lt::RouterPrep prep{drs, dpre, moe_in, inv_sqrt_d, eps};
    const float *rin = fuse_prep ? dx : router_in;
    if (!fuse_prep &&
        (rc = norm_run(ctx, 2, dx, nullptr, dpre, drs, moe_in, router_in, 1, (uint32_t)n, eps, inv_sqrt_d, flags)))
        return rc;
    // 417 routerTopKSoftmax, then the selected experts (463-479, GpuWeights.runExpertBatch)
    if ((rc = ensure(ctx, ctx->eh, (size_t)k * Kd * 4))) return rc;
    float *h = (float *)ctx->eh.p;
    const uint32_t norm = (flags & LT_MOE_NORM_TOPK) ? 1u : 0u;
    if (E <= kRoutedGateUpMaxExperts) {
        if ((rc = router_dev(ctx, R, rin, nullptr, 0, flags, nullptr, fuse_prep ? &prep : nullptr))) return rc;
        rc = gate_up_routed_dev(ctx, GU, moe_in, k, norm, d_expert, (uint32_t)Kd, act, h);
    } else {
        if ((rc = router_dev(ctx, R, rin, nullptr, k, flags, nullptr, fuse_prep ? &prep : nullptr))) return rc;
        rc = gate_up_dev(ctx, GU, moe_in, (const uint32_t *)ctx->ids.p, k, d_expert, (uint32_t)Kd, act, h);
    }
    if (rc) return rc;
    if ((rc = down_dev(ctx, D, h, (const uint32_t *)ctx->ids.p, (const float *)ctx->w.p, k, nullptr, 0, dds, moe)))
        return rc;
    // 482-497: post_ffw_norm_2, + dense FFN, post_ffw_norm, residual, layer_output_scale
    if ((rc = norm_run(ctx, 3, moe, dd, dp, dp2, xio, nullptr, 1, (uint32_t)n, eps, layer_output_scale, flags)))
        return rc;
    if ((rc = copy_routing_out(ctx, k, out_ids, out_w, host))) return rc;
    if (host) {
        LT_HIP(ctx, hipMemcpyAsync(x, xio, n * 4, hipMemcpyDeviceToHost, ctx->stream));
        LT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        prof_harvest(ctx);
    }
    return LT_OK;
}

// ------------------------------------------------------------------ profiling
extern "C" size_t lt_profile_report(lt_ctx *ctx, char *buf, size_t len) {
    if (!ctx || !ctx->prof.mode) {
        if (buf && len) buf[0] = 0;
        return 0;
    }
    Profile &P = ctx->prof;
    std::string o;
    char line[256];
    o += "LT_PROFILE spans: device time between HIP events around each call's work\n";
    snprintf(line, sizeof line, "%-34s %8s %12s %10s %10s %10s\n", "call", "count", "total ms", "mean us", "min us",
             "max us");
    o += line;
    for (const auto &kv : P.spans) {
        const SpanStat &st = kv.second;
        snprintf(line, sizeof line, "%-34s %8zu %12.3f %10.3f %10.3f %10.3f\n", kv.first.c_str(), st.n, st.total_ms,
                 st.n ? st.total_ms * 1e3 / st.n : 0.0, st.min_ms * 1e3, st.max_ms * 1e3);
        o += line;
    }
    if (P.mode == 2) {
        snprintf(line, sizeof line,
                 "\nLT_PROFILE timeline: single-launch MoE kernel, %zu launches (one per synchronising call);\n"
                 "us from the first block's start; median over launches of the block median / the last block\n",
                 P.launches);
        o += line;
        static const char *roles[kRoles] = {"", "router", "gate/up", "down", "combine", "sh g/u", "sh down", "tail"};
        static const char *phases[kRoles][kPhases] = {
            {},
            {"block start", "first row chunk in", "logit published", "all row terms in"},
            {"block start", "logits seen", "expert known", "dot products done", "h record published"},
            {"block start", "logits seen", "weight loads issued", "h records read", "adds issued",
             "shared h slice read", "shared rows added"},
            {"block start", "rows written"},
            {"block start", "h rows out"},
            {"block start", nullptr, nullptr, nullptr, nullptr, "h slice read", "rows added"},
            {"block start", "down blocks done", "x written"}};
        snprintf(line, sizeof line, "%-9s %-22s %10s %10s\n", "role", "phase", "median", "last");
        o += line;
        for (int r = 1; r < kRoles; r++)
            for (int ph = 0; ph < kPhases; ph++) {
                if (!phases[r][ph] || P.med[r][ph].empty()) continue;
                snprintf(line, sizeof line, "%-9s %-22s %10.2f %10.2f\n", roles[r], phases[r][ph], median_of(P.med[r][ph]),
                         median_of(P.last[r][ph]));
                o += line;
            }
        for (int r = 0; r < 2; r++) {
            o += r == 0 ? "gate/up h published, last block per slot:" : "down adds issued, last block per slot:   ";
            for (int q = 0; q < 16; q++)
                if (!P.slot_last[r][q].empty()) {
                    snprintf(line, sizeof line, " %d:%.2f", q, median_of(P.slot_last[r][q]));
                    o += line;
                }
            o += "\n";
        }
        if (!P.last_stamp.empty()) {
            snprintf(line, sizeof line, "last stamp of any block (median over launches): %.2f us\n", median_of(P.last_stamp));
            o += line;
        }
        snprintf(line, sizeof line, "XCD of block 0 per launch:");
        o += line;
        for (int q = 0; q < 8; q++)
            if (P.rot[q]) {
                snprintf(line, sizeof line, " %d:%zu", q, P.rot[q]);
                o += line;
            }
        snprintf(line, sizeof line, "; launches with a group (block index %% 8) on more than one XCD: %zu\n", P.split);
        o += line;
        if (!P.placement.empty()) o += P.placement;
    }
    if (buf && len) {
        const size_t n = o.size() < len - 1 ? o.size() : len - 1;
        memcpy(buf, o.data(), n);
        buf[n] = 0;
    }
    return o.size();
}
