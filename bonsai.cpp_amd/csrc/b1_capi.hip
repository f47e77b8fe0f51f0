// C ABI of the B1_0 linear (declared in include/bonsai_b1.h): argument
// checks, device checks, kernel dispatch, weight residency and the
// ggml-style custom-op callback.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <list>
#include <mutex>
#include <utility>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "bonsai_b1.h"
#include "b1_internal.h"

// The workspace of bonsai_b1_linear_f32_noalloc: one copy per device, held
// by the loaded code object until the process ends.  Host code never uses
// this name as an address (on the host it is only a handle for the runtime's
// symbol lookup); it uses the device address hipGetSymbolAddress returns for
// the current device, kept in DeviceInfo::scratch.
static __device__ __align__(256) uint8_t scratch[BONSAI_B1_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

constexpr int kWsFree = 8; // unpinned workspaces kept per device (about one per stream)

// A library-owned workspace of one stream.  `owner`: 0, or for the
// per-thread default stream (hipStreamPerThread, one handle value that names
// a different stream in every thread) the calling thread's id, so that two
// threads never share a buffer their streams do not order.  `pins`: handed
// out while the stream was being captured, so a graph may hold its address;
// a pinned buffer is never freed or evicted (growing allocates a new one),
// only bonsai_b1_release_workspaces frees it.  `users`: entry-point calls
// that hold it between the hand-out and their last launch; never evicted
// then (another thread may not free it under a call that has not launched
// yet).
struct Workspace {
    hipStream_t stream = nullptr;
    uint64_t owner = 0;
    void *ptr = nullptr;
    size_t bytes = 0;
    uint64_t last_use = 0;
    int pins = 0;
    int users = 0;
};

struct DeviceInfo {
    int state = 0; // 0 unknown, 1 usable gfx950, -1 unusable
    int num_cus = 0;
    std::list<Workspace> ws;       // stable element addresses
    uint64_t tick = 0;
    // this device's address of `scratch` (0: not looked up, 1: found, -1:
    // the lookup failed)
    int scratch_state = 0;
    void *scratch = nullptr;
};

std::mutex g_mu;
DeviceInfo g_dev[kMaxDevices];

// Looks up the current device's address of `scratch` (with that device
// current, under g_mu); nullptr when the lookup fails.
void lookup_scratch(DeviceInfo *d) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    d->scratch = e == hipSuccess ? p : nullptr;
    d->scratch_state = d->scratch ? 1 : -1;
}

// Returns the current device's info, probing it once.  The probe, which the
// first call of any entry point on a device makes, also looks up that
// device's copy of `scratch`.
DeviceInfo *current_device(int *dev_out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    if (dev_out) *dev_out = dev;
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceInfo &d = g_dev[dev];
    if (d.state == 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
            d.state = -1;
        } else {
            d.state = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
            d.num_cus = prop.multiProcessorCount;
            if (d.state == 1) lookup_scratch(&d);
        }
    }
    return d.state == 1 ? &d : nullptr;
}

// This device's address of `scratch` (nullptr if its lookup fails), with
// that device current.  A lookup that failed at the probe (say, while
// another stream of the process was being captured) is tried again here.
void *device_scratch(DeviceInfo *d) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (d->scratch_state != 1) lookup_scratch(d);
    return d->scratch_state == 1 ? d->scratch : nullptr;
}

// A library-owned workspace handed to one entry-point call, released (the
// user count dropped) when the call has launched its kernels.  ptr is
// nullptr when none could be had: the stream is being captured and owns no
// large enough buffer (a capture never allocates), or allocation failed, or
// every buffer is pinned or in use by another call.
class WsLease {
  public:
    WsLease() = default;
    WsLease(const WsLease &) = delete;
    WsLease &operator=(const WsLease &) = delete;
    ~WsLease() { drop(); }
    void *ptr() const { return w_ ? w_->ptr : nullptr; }
    void acquire(DeviceInfo *d, hipStream_t stream, size_t need);

  private:
    void drop() {
        if (w_) {
            std::lock_guard<std::mutex> lk(g_mu);
            --w_->users;
            w_ = nullptr;
        }
    }
    Workspace *w_ = nullptr;
};

// The workspace owner of a stream handle: the calling thread's id (from 1,
// never reused) for hipStreamPerThread, 0 for every other handle.
std::atomic<uint64_t> g_next_thread_id{0};
uint64_t stream_owner(hipStream_t stream) {
    if (stream != hipStreamPerThread) return 0;
    thread_local uint64_t id = 0;
    if (!id) id = g_next_thread_id.fetch_add(1) + 1;
    return id;
}

// Hands out this stream's most recently used buffer of at least `need`
// bytes (pinning it when the stream is being captured), or, outside a
// capture, a new one.  A new buffer takes the place of an unpinned buffer
// no call holds: this stream's own smaller one, or the least recently used
// one once kWsFree unpinned buffers exist; freeing waits for the device
// (hipFree), so work already launched on the old buffer completes first.
void WsLease::acquire(DeviceInfo *d, hipStream_t stream, size_t need) {
    drop();
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
    const uint64_t owner = stream_owner(stream);
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace *hit = nullptr;
    for (Workspace &w : d->ws)
        if (w.stream == stream && w.owner == owner && w.bytes >= need && (!hit || w.last_use > hit->last_use))
            hit = &w;
    if (hit) {
        hit->last_use = ++d->tick;
        ++hit->users;
        if (capturing) ++hit->pins;
        w_ = hit;
        return;
    }
    if (capturing) return;
    Workspace *own = nullptr, *lru = nullptr;
    int unpinned = 0;
    for (Workspace &w : d->ws) {
        if (w.pins) continue;
        ++unpinned;
        if (w.users) continue;
        if (w.stream == stream && w.owner == owner) own = &w;
        if (!lru || w.last_use < lru->last_use) lru = &w;
    }
    Workspace *slot = own ? own : unpinned >= kWsFree ? lru : nullptr;
    if (slot) {
        (void)hipFree(slot->ptr);
        slot->ptr = nullptr;
        slot->bytes = 0;
    }
    const size_t bytes = (need + (2u << 20) - 1) & ~((size_t)(2u << 20) - 1);
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        if (slot) d->ws.remove_if([slot](const Workspace &w) { return &w == slot; });
        return;
    }
    if (!slot) {
        d->ws.emplace_back();
        slot = &d->ws.back();
    }
    slot->stream = stream;
    slot->owner = owner;
    slot->ptr = p;
    slot->bytes = bytes;
    slot->last_use = ++d->tick;
    slot->pins = 0;
    slot->users = 1;
    w_ = slot;
}

int check_args(const float *act, int64_t lda, const void *w, int in_dim,
               int out_dim, int batch, const float *out, int64_t ldo) {
    if (in_dim <= 0 || out_dim <= 0 || batch < 0) return BONSAI_B1_ERR_ARG;
    if (in_dim % BONSAI_B1_BLOCK_SIZE != 0) return BONSAI_B1_ERR_ARG;
    if (lda < in_dim || ldo < out_dim) return BONSAI_B1_ERR_ARG;
    if (batch > 0 && (!act || !w || !out)) return BONSAI_B1_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(act) & 3u) || (reinterpret_cast<uintptr_t>(out) & 3u) ||
        (reinterpret_cast<uintptr_t>(w) & 1u))
        return BONSAI_B1_ERR_ARG;
    return BONSAI_B1_OK;
}

} // namespace

extern "C" {

int bonsai_b1_version(void) { return 100; }

const char *bonsai_b1_status_string(int status) {
    switch (status) {
    case BONSAI_B1_OK: return "ok";
    case BONSAI_B1_ERR_ARG: return "invalid argument";
    case BONSAI_B1_ERR_HIP: return "HIP runtime error";
    case BONSAI_B1_ERR_NONFINITE: return "non-finite output";
    case BONSAI_B1_ERR_DEVICE: return "no usable gfx950 device";
    case BONSAI_B1_ERR_NOT_FOUND: return "tensor not found";
    case BONSAI_B1_ERR_FORMAT: return "malformed file or not a B1_0 tensor";
    case BONSAI_B1_ERR_IO: return "file could not be opened";
    case BONSAI_B1_ERR_SCRATCH: return "call needs more workspace than the no-alloc scratch holds";
    default: return "unknown status";
    }
}

static b1::LinearArgs linear_args(const float *act, int64_t lda, const void *w, int in_dim, int out_dim, int batch,
                                  float *out, int64_t ldo, int32_t *nonfinite) {
    b1::LinearArgs a;
    a.act = act;
    a.lda = lda;
    a.w = static_cast<const uint8_t *>(w);
    a.K = in_dim;
    a.N = out_dim;
    a.M = batch;
    a.out = out;
    a.ldo = ldo;
    a.nonfinite = nonfinite;
    return a;
}

// The workspace the kernel linear_impl picks for these arguments can use:
// the FAST GEMM's range-safe packing and split-K partials; none for the
// small-M kernel and EXACT mode.
static size_t linear_need(const b1::LinearArgs &a, int mode, int num_cus) {
    if (mode == BONSAI_B1_MODE_EXACT || mode == BONSAI_B1_MODE_GEMV) return 0;
    if (mode != BONSAI_B1_MODE_GEMM && b1::gemv_supported(a)) return 0;
    return b1::gemm_supported(a) ? b1::gemm_workspace_bytes_total(a, num_cus) : 0;
}

// Shared body of the two linear entry points.  ws_mode: 0 = library-owned
// workspace, 1 = caller's (ws, ws_bytes; may be NULL / too small).
static int linear_impl(const float *act, int64_t lda, const void *w, int in_dim, int out_dim, int batch,
                       float *out, int64_t ldo, int mode, int32_t *nonfinite, int ws_mode, void *ws,
                       size_t ws_bytes, hipStream_t stream) {
    int st = check_args(act, lda, w, in_dim, out_dim, batch, out, ldo);
    if (st != BONSAI_B1_OK) return st;
    if (mode < BONSAI_B1_MODE_AUTO || mode > BONSAI_B1_MODE_GEMV) return BONSAI_B1_ERR_ARG;
    DeviceInfo *dev = current_device(nullptr);
    if (!dev) return BONSAI_B1_ERR_DEVICE;
    if (batch == 0) return BONSAI_B1_OK;

    const b1::LinearArgs a = linear_args(act, lda, w, in_dim, out_dim, batch, out, ldo, nonfinite);

    // the library's workspace for this stream (ws_mode 0), or the caller's
    WsLease lease;
    auto workspace = [&](size_t need) {
        if (need > 0 && ws_mode == 0) {
            lease.acquire(dev, stream, need);
            ws = lease.ptr();
            ws_bytes = ws ? need : 0;
        }
    };
    auto gemm = [&]() {
        workspace(linear_need(a, mode, dev->num_cus));
        return b1::launch_gemm(a, dev->num_cus, ws, ws_bytes, stream);
    };
    auto gemv = [&]() { return b1::launch_gemv(a, dev->num_cus, stream); };

    hipError_t e;
    switch (mode) {
    case BONSAI_B1_MODE_EXACT:
        e = b1::launch_exact(a, dev->num_cus, stream);
        break;
    case BONSAI_B1_MODE_GEMM:
        if (!b1::gemm_supported(a)) return BONSAI_B1_ERR_ARG;
        e = gemm();
        break;
    case BONSAI_B1_MODE_GEMV:
        if (!b1::gemv_supported(a)) return BONSAI_B1_ERR_ARG;
        e = gemv();
        break;
    default: // AUTO, FAST
        if (b1::gemv_supported(a))
            e = gemv();
        else if (b1::gemm_supported(a))
            e = gemm();
        else
            e = b1::launch_exact(a, dev->num_cus, stream); // unaligned / K % 64 != 0
        break;
    }
    return e == hipSuccess ? BONSAI_B1_OK : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_linear_f32(const float *act, int64_t lda, const void *w,
                         int in_dim, int out_dim, int batch, float *out,
                         int64_t ldo, int mode, int32_t *nonfinite,
                         hipStream_t stream) {
    return linear_impl(act, lda, w, in_dim, out_dim, batch, out, ldo, mode, nonfinite, 0, nullptr, 0, stream);
}

size_t bonsai_b1_workspace_bytes(int batch, int in_dim, int out_dim, int mode) {
    if (batch <= 0 || in_dim <= 0 || out_dim <= 0 || in_dim % BONSAI_B1_BLOCK_SIZE) return 0;
    if (mode < BONSAI_B1_MODE_AUTO || mode > BONSAI_B1_MODE_GEMV || mode == BONSAI_B1_MODE_EXACT) return 0;
    // the calls' own choice of kernel, on aligned activations
    b1::LinearArgs a{};
    a.K = in_dim;
    a.N = out_dim;
    a.M = batch;
    a.lda = in_dim;
    a.act = reinterpret_cast<const float *>(uintptr_t(256));
    a.w = reinterpret_cast<const uint8_t *>(uintptr_t(256));
    // the small-M kernel converts the activations itself
    if (mode == BONSAI_B1_MODE_GEMV || (mode != BONSAI_B1_MODE_GEMM && batch <= b1::kGemvMaxM)) return 0;
    // the range-safe packing, then (on a device where the shape splits
    // along K) the split-K partials
    const DeviceInfo *dev = current_device(nullptr);
    return b1::gemm_workspace_bytes_total(a, dev ? dev->num_cus : 0);
}

int bonsai_b1_linear_f32_ws(const float *act, int64_t lda, const void *w,
                            int in_dim, int out_dim, int batch, float *out,
                            int64_t ldo, int mode, int32_t *nonfinite,
                            void *workspace, size_t workspace_bytes,
                            hipStream_t stream) {
    return linear_impl(act, lda, w, in_dim, out_dim, batch, out, ldo, mode, nonfinite, 1, workspace,
                       workspace_bytes, stream);
}

int bonsai_b1_linear_f32_noalloc(const float *act, int64_t lda, const void *w, int in_dim, int out_dim, int batch,
                                 float *out, int64_t ldo, int mode, int32_t *nonfinite, hipStream_t stream) {
    // the argument checks of the shared body come first, so a bad call is
    // ERR_ARG whatever its size
    int st = check_args(act, lda, w, in_dim, out_dim, batch, out, ldo);
    if (st != BONSAI_B1_OK) return st;
    if (mode < BONSAI_B1_MODE_AUTO || mode > BONSAI_B1_MODE_GEMV) return BONSAI_B1_ERR_ARG;
    DeviceInfo *dev = current_device(nullptr);
    if (!dev) return BONSAI_B1_ERR_DEVICE;
    if (batch == 0) return BONSAI_B1_OK;
    // what the kernel this call runs would use (an unaligned call runs EXACT
    // mode and needs none)
    const b1::LinearArgs a = linear_args(act, lda, w, in_dim, out_dim, batch, out, ldo, nonfinite);
    if (linear_need(a, mode, dev->num_cus) > BONSAI_B1_NOALLOC_SCRATCH_BYTES) return BONSAI_B1_ERR_SCRATCH;
    void *ws = device_scratch(dev);
    if (!ws) return BONSAI_B1_ERR_HIP;
    return linear_impl(act, lda, w, in_dim, out_dim, batch, out, ldo, mode, nonfinite, 1, ws,
                       BONSAI_B1_NOALLOC_SCRATCH_BYTES, stream);
}

int bonsai_b1_gelu_tanh_f32(const float *x, int64_t ldx, float *y, int64_t ldy, int cols, int rows,
                            hipStream_t stream) {
    if (cols < 0 || rows < 0 || cols % 4 || ldx < cols || ldy < cols || ldx % 4 || ldy % 4) return BONSAI_B1_ERR_ARG;
    if (rows > 0 && cols > 0 && (!x || !y)) return BONSAI_B1_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(y) & 15u)) return BONSAI_B1_ERR_ARG;
    if (!current_device(nullptr)) return BONSAI_B1_ERR_DEVICE;
    if (rows == 0 || cols == 0) return BONSAI_B1_OK;
    return b1::launch_gelu(x, ldx, y, ldy, cols, rows, stream) == hipSuccess ? BONSAI_B1_OK : BONSAI_B1_ERR_HIP;
}

// Arguments of the packing producers: packed rows of ldp fp16 elements
// (ldp >= in_dim, 16-byte row alignment), packed 16-byte aligned.
static int pack_args(const float *act, int64_t lda, int in_dim, int batch, const void *packed, int64_t ldp) {
    if (in_dim <= 0 || batch < 0 || in_dim % BONSAI_B1_BLOCK_SIZE || lda < in_dim) return BONSAI_B1_ERR_ARG;
    if (ldp < in_dim || ldp % 8) return BONSAI_B1_ERR_ARG;
    if (batch > 0 && (!act || !packed)) return BONSAI_B1_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(packed) & 15u) return BONSAI_B1_ERR_ARG;
    if (batch > 0 && !b1::pack_supported(act, lda, batch, in_dim)) return BONSAI_B1_ERR_ARG;
    if (!current_device(nullptr)) return BONSAI_B1_ERR_DEVICE;
    return BONSAI_B1_OK;
}

int bonsai_b1_gelu_tanh_pack_f16_ld(const float *act, int64_t lda, int in_dim, int batch, void *packed,
                                    int64_t ldp, hipStream_t stream) {
    const int st = pack_args(act, lda, in_dim, batch, packed, ldp);
    if (st != BONSAI_B1_OK || batch == 0) return st;
    return b1::launch_gelu_pack(act, lda, batch, in_dim, packed, ldp, stream) == hipSuccess ? BONSAI_B1_OK
                                                                                           : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_gelu_tanh_pack_f16(const float *act, int64_t lda, int in_dim, int batch, void *packed,
                                 hipStream_t stream) {
    return bonsai_b1_gelu_tanh_pack_f16_ld(act, lda, in_dim, batch, packed, in_dim, stream);
}

int bonsai_b1_swiglu_pack_f16_ld(const float *act, int64_t lda, int hidden, int batch, void *packed, int64_t ldp,
                                 hipStream_t stream) {
    if (hidden <= 0 || hidden % BONSAI_B1_BLOCK_SIZE || hidden > INT32_MAX / 2) return BONSAI_B1_ERR_ARG;
    if (ldp < hidden || ldp % 8) return BONSAI_B1_ERR_ARG;
    // the input as a pack of its 2 hidden columns would be checked; the
    // output row stride is checked above
    const int st = pack_args(act, lda, 2 * hidden, batch, packed, 2 * hidden);
    if (st != BONSAI_B1_OK || batch == 0) return st;
    return b1::launch_swiglu_pack(act, lda, batch, hidden, packed, ldp, stream) == hipSuccess ? BONSAI_B1_OK
                                                                                             : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_swiglu_pack_f16(const float *act, int64_t lda, int hidden, int batch, void *packed,
                              hipStream_t stream) {
    return bonsai_b1_swiglu_pack_f16_ld(act, lda, hidden, batch, packed, hidden, stream);
}

static int norm_mod_args(const float *x, int64_t ldx, int H, int rows, const float *scale, const float *shift,
                         const void *dst) {
    auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (H <= 0 || rows < 0 || H % BONSAI_B1_BLOCK_SIZE || ldx < H || ldx % 4) return BONSAI_B1_ERR_ARG;
    if (rows > 0 && (!x || !scale || !shift || !dst)) return BONSAI_B1_ERR_ARG;
    if (!al16(x) || !al16(scale) || !al16(shift) || !al16(dst)) return BONSAI_B1_ERR_ARG;
    if ((uint64_t)rows * (uint64_t)H >= (1ull << 40)) return BONSAI_B1_ERR_ARG;
    return BONSAI_B1_OK;
}

int bonsai_b1_norm_mod_f32(const float *x, int64_t ldx, int H, int rows, const float *scale, const float *shift,
                           float eps, float *y, int64_t ldy, hipStream_t stream) {
    int st = norm_mod_args(x, ldx, H, rows, scale, shift, y);
    if (st != BONSAI_B1_OK) return st;
    if (ldy < H || ldy % 4) return BONSAI_B1_ERR_ARG;
    if (!current_device(nullptr)) return BONSAI_B1_ERR_DEVICE;
    if (rows == 0) return BONSAI_B1_OK;
    return b1::launch_norm_mod(x, ldx, H, rows, scale, shift, eps, y, ldy, nullptr, stream) == hipSuccess
               ? BONSAI_B1_OK
               : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_norm_mod_pack_f16(const float *x, int64_t ldx, int H, int rows, const float *scale,
                                const float *shift, float eps, void *packed, hipStream_t stream) {
    int st = norm_mod_args(x, ldx, H, rows, scale, shift, packed);
    if (st != BONSAI_B1_OK) return st;
    if (!current_device(nullptr)) return BONSAI_B1_ERR_DEVICE;
    if (rows == 0) return BONSAI_B1_OK;
    return b1::launch_norm_mod(x, ldx, H, rows, scale, shift, eps, nullptr, 0, packed, stream) == hipSuccess
               ? BONSAI_B1_OK
               : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_quantize_f32(const float *w, int64_t ldw, int in_dim, int out_dim, void *packed, int order,
                           hipStream_t stream) {
    if (in_dim <= 0 || out_dim < 0 || in_dim % BONSAI_B1_BLOCK_SIZE || ldw < in_dim) return BONSAI_B1_ERR_ARG;
    if (order != BONSAI_B1_SUM_NUMPY && order != BONSAI_B1_SUM_SEQUENTIAL) return BONSAI_B1_ERR_ARG;
    if (out_dim > 0 && (!w || !packed)) return BONSAI_B1_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(w) & 3u) || (reinterpret_cast<uintptr_t>(packed) & 1u)) return BONSAI_B1_ERR_ARG;
    if (!current_device(nullptr)) return BONSAI_B1_ERR_DEVICE;
    if (out_dim == 0) return BONSAI_B1_OK;
    return b1::launch_quantize(w, ldw, in_dim, out_dim, packed, order, stream) == hipSuccess ? BONSAI_B1_OK
                                                                                            : BONSAI_B1_ERR_HIP;
}

size_t bonsai_b1_packed_act_bytes(int batch, int in_dim) {
    if (batch <= 0 || in_dim <= 0 || in_dim % BONSAI_B1_BLOCK_SIZE) return 0;
    return (size_t)batch * (size_t)in_dim * 2;
}

int bonsai_b1_pack_act_f16_ld(const float *act, int64_t lda, int in_dim, int batch, void *packed, int64_t ldp,
                              hipStream_t stream) {
    const int st = pack_args(act, lda, in_dim, batch, packed, ldp);
    if (st != BONSAI_B1_OK || batch == 0) return st;
    return b1::launch_pack(act, lda, batch, in_dim, packed, ldp, stream) == hipSuccess ? BONSAI_B1_OK
                                                                                      : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_pack_act_f16(const float *act, int64_t lda, int in_dim, int batch, void *packed,
                           hipStream_t stream) {
    return bonsai_b1_pack_act_f16_ld(act, lda, in_dim, batch, packed, in_dim, stream);
}

int bonsai_b1_pack_act_f16_scaled(const float *act, int64_t lda, int in_dim, int batch, void *packed,
                                  float *row_scale, hipStream_t stream) {
    if (batch > 0 && (!row_scale || (reinterpret_cast<uintptr_t>(row_scale) & 3u))) return BONSAI_B1_ERR_ARG;
    const int st = pack_args(act, lda, in_dim, batch, packed, in_dim);
    if (st != BONSAI_B1_OK || batch == 0) return st;
    return b1::launch_pack_rows_to(act, lda, batch, in_dim, packed, row_scale, stream) == hipSuccess
               ? BONSAI_B1_OK
               : BONSAI_B1_ERR_HIP;
}

size_t bonsai_b1_linear_packed_workspace_bytes(int batch, int in_dim, int out_dim) {
    if (batch <= 0 || in_dim <= 0 || out_dim <= 0 || !b1::gemm_packed_ok(batch, in_dim, out_dim)) return 0;
    if (b1::gemv_packed_ok(batch, in_dim, out_dim)) return 0;
    const DeviceInfo *dev = current_device(nullptr);
    const int splits = dev ? b1::gemm_splits(batch, in_dim, out_dim, dev->num_cus) : 1;
    return b1::gemm_split_bytes(batch, out_dim, splits);
}

// Shared body of the packed entry points.  ws_mode: 0 = library-owned
// workspace for the split-K partials, 1 = caller's (may be NULL / small:
// then unsplit).
static int linear_packed_impl(const void *packed_act, const float *rsc, const void *w, int in_dim, int out_dim,
                              int batch, float *out, int64_t ldo, int32_t *nonfinite, int ws_mode, void *ws,
                              size_t ws_bytes, hipStream_t stream) {
    if (in_dim <= 0 || out_dim <= 0 || batch < 0 || ldo < out_dim) return BONSAI_B1_ERR_ARG;
    if (batch > 0 && (!packed_act || !w || !out)) return BONSAI_B1_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(packed_act) & 15u) || (reinterpret_cast<uintptr_t>(w) & 3u) ||
        (reinterpret_cast<uintptr_t>(out) & 3u) || (reinterpret_cast<uintptr_t>(ws) & 15u) ||
        (reinterpret_cast<uintptr_t>(rsc) & 3u))
        return BONSAI_B1_ERR_ARG;
    if (!b1::gemm_packed_ok(batch > 0 ? batch : 1, in_dim, out_dim)) return BONSAI_B1_ERR_ARG;
    DeviceInfo *dev = current_device(nullptr);
    if (!dev) return BONSAI_B1_ERR_DEVICE;
    if (batch == 0) return BONSAI_B1_OK;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    hipError_t e;
    if (b1::gemv_packed_ok(batch, in_dim, out_dim)) {
        // a few tokens: the bandwidth-bound small-M kernel, not a 128-row tile
        e = b1::launch_gemv_packed(packed_act, wb, in_dim, out_dim, batch, out, ldo, nonfinite, dev->num_cus, stream,
                                   rsc);
    } else {
        // split along K as bonsai_b1_linear_f32 splits the same shape, when
        // the partials have room: the two entries then agree bit for bit
        const int splits = b1::gemm_splits(batch, in_dim, out_dim, dev->num_cus);
        const size_t need = b1::gemm_split_bytes(batch, out_dim, splits);
        WsLease lease;
        if (need > 0 && ws_mode == 0) {
            lease.acquire(dev, stream, need);
            ws = lease.ptr();
            ws_bytes = ws ? need : 0;
        }
        b1::GemmEpi epi;
        epi.rsc = rsc;
        if (need > 0 && ws && ws_bytes >= need)
            e = b1::launch_gemm_packed_split(packed_act, wb, in_dim, out_dim, batch, out, ldo, nonfinite,
                                             dev->num_cus, splits, ws, stream, rsc);
        else
            e = b1::launch_gemm_packed_epi(packed_act, wb, in_dim, out_dim, batch, out, ldo, nonfinite, dev->num_cus,
                                           0, epi, stream);
    }
    return e == hipSuccess ? BONSAI_B1_OK : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_linear_packed_f16_scaled(const void *packed_act, const float *row_scale, const void *w, int in_dim,
                                       int out_dim, int batch, float *out, int64_t ldo, int32_t *nonfinite,
                                       hipStream_t stream) {
    if (batch > 0 && !row_scale) return BONSAI_B1_ERR_ARG;
    return linear_packed_impl(packed_act, row_scale, w, in_dim, out_dim, batch, out, ldo, nonfinite, 0, nullptr, 0,
                              stream);
}

int bonsai_b1_linear_packed_f16(const void *packed_act, const void *w, int in_dim, int out_dim, int batch,
                                float *out, int64_t ldo, int32_t *nonfinite, hipStream_t stream) {
    return linear_packed_impl(packed_act, nullptr, w, in_dim, out_dim, batch, out, ldo, nonfinite, 0, nullptr, 0,
                              stream);
}

int bonsai_b1_linear_packed_f16_ws(const void *packed_act, const void *w, int in_dim, int out_dim, int batch,
                                   float *out, int64_t ldo, int32_t *nonfinite, void *workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
    return linear_packed_impl(packed_act, nullptr, w, in_dim, out_dim, batch, out, ldo, nonfinite, 1, workspace,
                              workspace_bytes, stream);
}

// Checks an epilogue against a linear of out_dim outputs (weight rows) and
// fills the kernels' form.  out's row length is out_dim, or out_dim / 2
// for SwiGLU.
static int epi_args(const bonsai_b1_epilogue *epi, int out_dim, int batch, const float *out, int64_t ldo, int *kind,
                    b1::GemmEpi *g) {
    *kind = epi ? epi->kind : BONSAI_B1_EPI_NONE;
    *g = b1::GemmEpi();
    auto span = [](const float *p, int rows, int64_t ld, int cols) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(p);
        return std::pair<uintptr_t, uintptr_t>(a, a + ((size_t)(rows - 1) * (size_t)ld + (size_t)cols) * 4);
    };
    auto overlap = [](std::pair<uintptr_t, uintptr_t> x, std::pair<uintptr_t, uintptr_t> y) {
        return x.first < y.second && y.first < x.second;
    };
    switch (*kind) {
    case BONSAI_B1_EPI_NONE:
        return ldo >= out_dim ? BONSAI_B1_OK : BONSAI_B1_ERR_ARG;
    case BONSAI_B1_EPI_GATE_RESIDUAL: {
        if (ldo < out_dim || epi->ldr < out_dim) return BONSAI_B1_ERR_ARG;
        if (batch > 0) {
            if (!epi->gate || !epi->residual) return BONSAI_B1_ERR_ARG;
            if ((reinterpret_cast<uintptr_t>(epi->gate) & 3u) || (reinterpret_cast<uintptr_t>(epi->residual) & 3u))
                return BONSAI_B1_ERR_ARG;
            const auto o = span(out, batch, ldo, out_dim);
            // the residual is out itself (read and written element by
            // element) or lies apart from it; the gate lies apart
            if (epi->residual == out) {
                if (epi->ldr != ldo) return BONSAI_B1_ERR_ARG;
            } else if (overlap(o, span(epi->residual, batch, epi->ldr, out_dim))) {
                return BONSAI_B1_ERR_ARG;
            }
            if (overlap(o, span(epi->gate, 1, out_dim, out_dim))) return BONSAI_B1_ERR_ARG;
        }
        g->gate = epi->gate;
        g->res = epi->residual;
        g->ldr = epi->ldr;
        return BONSAI_B1_OK;
    }
    case BONSAI_B1_EPI_SWIGLU:
        if (out_dim % 64 != 0 || ldo < out_dim / 2) return BONSAI_B1_ERR_ARG;
        g->glu_h = out_dim / 2;
        return BONSAI_B1_OK;
    case BONSAI_B1_EPI_PACKED: {
        const int split = epi->split, act = epi->act;
        if (split < 0 || split > out_dim || split % BONSAI_B1_BLOCK_SIZE || out_dim % BONSAI_B1_BLOCK_SIZE)
            return BONSAI_B1_ERR_ARG;
        if (act != BONSAI_B1_ACT_NONE && act != BONSAI_B1_ACT_GELU_TANH && act != BONSAI_B1_ACT_SWIGLU)
            return BONSAI_B1_ERR_ARG;
        const bool glu = act == BONSAI_B1_ACT_SWIGLU;
        if (glu && (split % 64 || (out_dim - split) % 64)) return BONSAI_B1_ERR_ARG;
        // packed columns written: SwiGLU halves its [gate | value] columns
        const int pcols = glu ? (out_dim - split) / 2 : out_dim - split;
        auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
        if (split > 0 && (!al16(out) || ldo < split || ldo % 4)) return BONSAI_B1_ERR_ARG;
        if (pcols > 0 && (!al16(epi->packed) || epi->ldp < pcols || epi->ldp % 8)) return BONSAI_B1_ERR_ARG;
        if (batch > 0) {
            if ((split > 0 && !out) || (pcols > 0 && !epi->packed)) return BONSAI_B1_ERR_ARG;
            if (split > 0 && pcols > 0) {
                const uintptr_t p0 = reinterpret_cast<uintptr_t>(epi->packed);
                const auto po = std::pair<uintptr_t, uintptr_t>(
                    p0, p0 + ((size_t)(batch - 1) * (size_t)epi->ldp + (size_t)pcols) * 2);
                if (overlap(po, span(out, batch, ldo, split))) return BONSAI_B1_ERR_ARG;
            }
        }
        g->pk = static_cast<uint32_t *>(epi->packed);
        g->ldpw = epi->ldp / 2;
        g->split = split;
        g->act = act;
        g->glu_h = glu ? pcols : 0;
        return BONSAI_B1_OK;
    }
    default:
        return BONSAI_B1_ERR_ARG;
    }
}

int bonsai_b1_linear_packed_f16_epi(const void *packed_act, const void *w, int in_dim, int out_dim, int batch,
                                    float *out, int64_t ldo, const bonsai_b1_epilogue *epi, int32_t *nonfinite,
                                    hipStream_t stream) {
    if (in_dim <= 0 || out_dim <= 0 || batch < 0) return BONSAI_B1_ERR_ARG;
    if (batch > 0 && (!packed_act || !w || !out)) return BONSAI_B1_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(packed_act) & 15u) || (reinterpret_cast<uintptr_t>(w) & 3u) ||
        (reinterpret_cast<uintptr_t>(out) & 3u))
        return BONSAI_B1_ERR_ARG;
    int kind;
    b1::GemmEpi g;
    int st = epi_args(epi, out_dim, batch, out, ldo, &kind, &g);
    if (st != BONSAI_B1_OK) return st;
    if (!b1::gemm_packed_ok(batch > 0 ? batch : 1, in_dim, out_dim)) return BONSAI_B1_ERR_ARG;
    DeviceInfo *dev = current_device(nullptr);
    if (!dev) return BONSAI_B1_ERR_DEVICE;
    if (batch == 0) return BONSAI_B1_OK;
    return b1::launch_gemm_packed_epi(packed_act, static_cast<const uint8_t *>(w), in_dim, out_dim, batch, out, ldo,
                                      nonfinite, dev->num_cus, kind, g, stream) == hipSuccess
               ? BONSAI_B1_OK
               : BONSAI_B1_ERR_HIP;
}

int bonsai_b1_linear_packed_f16_to_packed(const void *packed_act, const void *w, int in_dim, int out_dim, int batch,
                                          float *out, int64_t ldo, int split, int act, void *packed_out,
                                          int64_t ldp, int32_t *nonfinite, hipStream_t stream) {
    if (in_dim <= 0 || out_dim <= 0 || batch < 0) return BONSAI_B1_ERR_ARG;
    bonsai_b1_epilogue e = {};
    e.kind = BONSAI_B1_EPI_PACKED;
    e.split = split;
    e.act = act;
    e.packed = packed_out;
    e.ldp = ldp;
    int kind;
    b1::GemmEpi g;
    const int st = epi_args(&e, out_dim, batch, out, ldo, &kind, &g);
    if (st != BONSAI_B1_OK) return st;
    if ((reinterpret_cast<uintptr_t>(packed_act) & 15u) || (reinterpret_cast<uintptr_t>(w) & 3u))
        return BONSAI_B1_ERR_ARG;
    if (!b1::gemm_packed_ok(batch > 0 ? batch : 1, in_dim, out_dim)) return BONSAI_B1_ERR_ARG;
    if (batch > 0) {
        if (!packed_act || !w) return BONSAI_B1_ERR_ARG;
        // the outputs lie apart from the activations the GEMM still reads
        const uintptr_t a0 = reinterpret_cast<uintptr_t>(packed_act);
        const uintptr_t a1 = a0 + (size_t)batch * (size_t)in_dim * 2;
        auto apart = [&](const void *p, int64_t ld_bytes, int64_t row_bytes) {
            const uintptr_t p0 = reinterpret_cast<uintptr_t>(p);
            const uintptr_t p1 = p0 + (size_t)(batch - 1) * (size_t)ld_bytes + (size_t)row_bytes;
            return !(p0 < a1 && a0 < p1);
        };
        const int pcols = g.glu_h ? g.glu_h : out_dim - split;
        if (split > 0 && !apart(out, ldo * 4, (int64_t)split * 4)) return BONSAI_B1_ERR_ARG;
        if (pcols > 0 && !apart(packed_out, ldp * 2, (int64_t)pcols * 2)) return BONSAI_B1_ERR_ARG;
    }
    DeviceInfo *dev = current_device(nullptr);
    if (!dev) return BONSAI_B1_ERR_DEVICE;
    if (batch == 0) return BONSAI_B1_OK;
    return b1::launch_gemm_packed_epi(packed_act, static_cast<const uint8_t *>(w), in_dim, out_dim, batch, out, ldo,
                                      nonfinite, dev->num_cus, kind, g, stream) == hipSuccess
               ? BONSAI_B1_OK
               : BONSAI_B1_ERR_HIP;
}

// The fp32 output of a linear whose epilogue runs as a separate pass, in a
// workspace (256-byte multiple, so what follows stays aligned).
static size_t epi_y_bytes(int batch, int out_dim) { return ((size_t)batch * out_dim * 4 + 255) & ~(size_t)255; }

// Whether a linear runs the packed FAST GEMM (as linear_impl decides).
static bool packed_path(const b1::LinearArgs &a, int mode) {
    if (mode == BONSAI_B1_MODE_EXACT || mode == BONSAI_B1_MODE_GEMV) return false;
    if (mode != BONSAI_B1_MODE_GEMM && b1::gemv_supported(a)) return false;
    return b1::gemm_supported(a) && b1::gemm_workspace_bytes(a) > 0 && b1::pack_supported(a.act, a.lda, a.M, a.K);
}

size_t bonsai_b1_linear_epi_workspace_bytes(int batch, int in_dim, int out_dim, int kind, int mode) {
    if (batch <= 0 || in_dim <= 0 || out_dim <= 0 || in_dim % BONSAI_B1_BLOCK_SIZE) return 0;
    if (kind == BONSAI_B1_EPI_NONE) return bonsai_b1_workspace_bytes(batch, in_dim, out_dim, mode);
    // either the range-safe packing (fused path) or the linear's fp32 output
    // (separate pass; the linear then runs a kernel that needs no workspace
    // of its own)
    const size_t pack = b1::gemm_packed_ok(batch, in_dim, out_dim) ? b1::pack_area_bytes(batch, in_dim) : 0;
    const size_t y = epi_y_bytes(batch, out_dim);
    return pack > y ? pack : y;
}

int bonsai_b1_linear_epi_f32(const float *act, int64_t lda, const void *w, int in_dim, int out_dim, int batch,
                             float *out, int64_t ldo, const bonsai_b1_epilogue *epi, int mode, int32_t *nonfinite,
                             void *workspace, size_t workspace_bytes, hipStream_t stream) {
    int kind;
    b1::GemmEpi g;
    int st = epi_args(epi, out_dim, batch, out, ldo, &kind, &g);
    if (st != BONSAI_B1_OK) return st;
    if (kind == BONSAI_B1_EPI_NONE)
        return linear_impl(act, lda, w, in_dim, out_dim, batch, out, ldo, mode, nonfinite, workspace ? 1 : 0,
                           workspace, workspace_bytes, stream);
    // (the packed-output epilogue's out may be NULL: its checks are done)
    const bool packed_out = kind == BONSAI_B1_EPI_PACKED;
    st = check_args(act, lda, w, in_dim, out_dim, batch, packed_out ? act : out, out_dim);
    if (st != BONSAI_B1_OK) return st;
    if (mode < BONSAI_B1_MODE_AUTO || mode > BONSAI_B1_MODE_GEMV) return BONSAI_B1_ERR_ARG;
    DeviceInfo *dev = current_device(nullptr);
    if (!dev) return BONSAI_B1_ERR_DEVICE;
    if (batch == 0) return BONSAI_B1_OK;
    const b1::LinearArgs a = linear_args(act, lda, w, in_dim, out_dim, batch, out, ldo, nonfinite);
    const bool fused = packed_path(a, mode);
    // separate pass: y, then what the linear's own kernel can use
    const size_t y_bytes = epi_y_bytes(batch, out_dim);
    const size_t need = fused ? b1::pack_area_bytes(batch, in_dim) : y_bytes;
    WsLease lease;
    if (!workspace) {
        lease.acquire(dev, stream, need);
        workspace = lease.ptr();
        workspace_bytes = workspace ? need : 0;
    }
    if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
        return BONSAI_B1_ERR_ARG;
    if (packed_out) {
        // the outputs lie apart from the workspace the GEMM or the
        // separate passes read
        const uintptr_t w0 = reinterpret_cast<uintptr_t>(workspace), w1 = w0 + need;
        auto apart = [&](const void *p, size_t bytes) {
            const uintptr_t p0 = reinterpret_cast<uintptr_t>(p);
            return bytes == 0 || !(p0 < w1 && w0 < p0 + bytes);
        };
        const int pcols = g.glu_h ? g.glu_h : out_dim - g.split;
        if (!apart(out, g.split ? ((size_t)(batch - 1) * ldo + g.split) * 4 : 0) ||
            !apart(epi->packed, pcols ? ((size_t)(batch - 1) * epi->ldp + pcols) * 2 : 0))
            return BONSAI_B1_ERR_ARG;
    }
    hipError_t e;
    if (fused) {
        e = b1::launch_pack_rows(act, lda, batch, in_dim, workspace, stream);
        g.rsc = b1::pack_area_rsc(workspace, batch, in_dim);
        if (e == hipSuccess)
            e = b1::launch_gemm_packed_epi(workspace, a.w, in_dim, out_dim, batch, out, ldo, nonfinite, dev->num_cus,
                                           kind, g, stream);
    } else {
        // the linear into the workspace (a kernel that needs no workspace of
        // its own), then the epilogue pass
        float *y = static_cast<float *>(workspace);
        st = linear_impl(act, lda, w, in_dim, out_dim, batch, y, out_dim, mode, nonfinite, 1, nullptr, 0, stream);
        if (st != BONSAI_B1_OK) return st;
        e = packed_out ? b1::launch_epi_packed(y, out_dim, batch, out_dim, g, out, ldo, stream)
                       : b1::launch_epi(y, out_dim, batch, out_dim, kind, g, out, ldo, stream);
    }
    return e == hipSuccess ? BONSAI_B1_OK : BONSAI_B1_ERR_HIP;
}

void bonsai_b1_release_workspaces(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (DeviceInfo &d : g_dev) {
        // buffers an unfinished call still holds stay (it frees nothing it
        // has not launched on yet); pinned ones go, as documented
        d.ws.remove_if([](Workspace &w) {
            if (w.users) return false;
            (void)hipFree(w.ptr);
            return true;
        });
    }
}

// How one op of a batch runs (the same choice linear_impl makes).
// Gemv: the small-M kernel (converting fp32 itself, or over the batch's
// range-safe packing when it runs in a group, gemv_span); Packed: the packed
// GEMM; Fused: the fused-conversion GEMM.
enum class BatchPath { Exact, Gemv, Packed, Fused };

static BatchPath batch_path(const b1::LinearArgs &a, int mode) {
    if (mode == BONSAI_B1_MODE_EXACT) return BatchPath::Exact;
    if (b1::gemv_supported(a)) return BatchPath::Gemv;
    if (b1::gemm_supported(a))
        return b1::gemm_workspace_bytes(a) > 0 ? BatchPath::Packed : BatchPath::Fused;
    return BatchPath::Exact;
}

static b1::LinearArgs batch_args(const bonsai_b1_linear_op &op) {
    b1::LinearArgs a;
    a.act = op.act;
    a.lda = op.lda;
    a.w = static_cast<const uint8_t *>(op.w->data);
    a.K = op.w->in_dim;
    a.N = op.w->out_dim;
    a.M = op.batch;
    a.out = op.out;
    a.ldo = op.ldo;
    a.nonfinite = nullptr;
    return a;
}

// The op's own arguments; out's row stride is checked against out_dim
// columns, or out_dim / 2 after SwiGLU (epi_args checks that case).
static bool batch_op_ok(const bonsai_b1_linear_op &op, const bonsai_b1_epilogue *epi = nullptr) {
    if (!op.w || !op.w->data) return false;
    // the SwiGLU and packed-output epilogues check their outputs themselves
    // (epi_args): out may be narrower, or NULL for a wholly packed output
    const bool own = epi && (epi->kind == BONSAI_B1_EPI_SWIGLU || epi->kind == BONSAI_B1_EPI_PACKED);
    const float *out = epi && epi->kind == BONSAI_B1_EPI_PACKED ? op.act : op.out;
    return check_args(op.act, op.lda, op.w->data, op.w->in_dim, op.w->out_dim, op.batch, out,
                      own ? op.w->out_dim : op.ldo) == BONSAI_B1_OK;
}

extern "C++" {

// One op of a batch and its epilogue (nullptr: none).
struct BatchOp {
    const bonsai_b1_linear_op *op;
    const bonsai_b1_epilogue *epi;
};

static int epi_kind(const bonsai_b1_epilogue *e) { return e ? e->kind : BONSAI_B1_EPI_NONE; }

static size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// The ops from i on that run as one GEMM with op i, on the packed path:
// consecutive plain ops on the same input whose weights follow each other in
// memory and whose outputs are adjacent column ranges of one row stride (q/k/v
// with concatenated weights, src/diffuser_graph.cpp:354-361), split along K
// as op i alone would be, unless an output overlaps the input they all read.
// Returns the last op of the run; *n_sum is its output width.
template <class OpAt>
static int fuse_span(int n_ops, int mode, int num_cus, OpAt at, int i, int *n_sum) {
    const BatchOp bi = at(i);
    const b1::LinearArgs a = batch_args(*bi.op);
    const int splits = b1::gemm_splits(a.M, a.K, a.N, num_cus);
    int last = i;
    *n_sum = a.N;
    while (epi_kind(bi.epi) == BONSAI_B1_EPI_NONE && last + 1 < n_ops) {
        const BatchOp pb = at(last), qb = at(last + 1);
        const bonsai_b1_linear_op &p = *pb.op, &q = *qb.op;
        if (!batch_op_ok(q, qb.epi)) break;
        // the packed size from the dimensions (nbytes is not trusted)
        const size_t p_bytes =
            (size_t)p.w->out_dim * (size_t)(p.w->in_dim / BONSAI_B1_BLOCK_SIZE) * BONSAI_B1_BLOCK_BYTES;
        if (epi_kind(qb.epi) != BONSAI_B1_EPI_NONE || q.batch != a.M || q.act != a.act || q.lda != a.lda ||
            q.w->in_dim != a.K || q.ldo != a.ldo || q.w->data != static_cast<const uint8_t *>(p.w->data) + p_bytes ||
            q.out != p.out + p.w->out_dim || *n_sum + (int64_t)q.w->out_dim > INT32_MAX ||
            !b1::gemm_packed_ok(a.M, a.K, *n_sum + q.w->out_dim))
            break;
        const b1::LinearArgs qa = batch_args(q);
        if (batch_path(qa, mode) != BatchPath::Packed || b1::gemm_splits(qa.M, qa.K, qa.N, num_cus) != splits) break;
        // the concatenated GEMM runs the tile kernel each part would (the
        // two sum K in different orders)
        const int tk = b1::gemm_tiles(a.M, a.K, a.N, num_cus);
        if (b1::gemm_tiles(qa.M, qa.K, qa.N, num_cus) != tk ||
            b1::gemm_tiles(a.M, a.K, *n_sum + q.w->out_dim, num_cus) != tk)
            break;
        *n_sum += q.w->out_dim;
        ++last;
    }
    if (last > i) {
        const uintptr_t o0 = reinterpret_cast<uintptr_t>(a.out);
        const uintptr_t o1 = o0 + ((size_t)(a.M - 1) * (size_t)a.ldo + (size_t)*n_sum) * sizeof(float);
        const uintptr_t i0 = reinterpret_cast<uintptr_t>(a.act);
        const uintptr_t i1 = i0 + ((size_t)(a.M - 1) * (size_t)a.lda + (size_t)a.K) * sizeof(float);
        if (o0 < i1 && i0 < o1) {
            last = i;
            *n_sum = a.N;
        }
    }
    return last;
}

// A grouped small-M run of at most kGemvGroupF32MaxM (8) tokens reads their
// fp32 rows itself (no packing, outputs equal to the single calls bit for
// bit, out-of-range tokens included); a larger one reads a range-safe
// packing.
static bool gemv_group_direct(const b1::LinearArgs &a) {
    return a.M <= b1::kGemvGroupF32MaxM && b1::gemv_group_f32_ok(a.act, a.lda, a.M, a.K);
}

// The ops from i on that run as one grouped small-M launch with op i:
// consecutive plain small-M ops on the same input (the modulation
// projections of src/diffuser_graph.cpp:308-311, 470-471 and 548 all read
// vec_silu at one token), at most kGemvGroupMax, whose outputs lie apart
// from that input and from one another (the group writes them in no
// particular order).  Returns the last op of the run, i when op i runs
// alone; fills ops[0 .. last - i].  pack_groups: a run that would read a
// packing (more than kGemvGroupF32MaxM tokens) may form; when false (no
// workspace to be had) its ops run one by one.
template <class OpAt>
static int gemv_span(int n_ops, int mode, OpAt at, int i, b1::GemvGroupOp *ops, bool pack_groups) {
    const BatchOp bi = at(i);
    const b1::LinearArgs a = batch_args(*bi.op);
    if (epi_kind(bi.epi) != BONSAI_B1_EPI_NONE || batch_path(a, mode) != BatchPath::Gemv ||
        !(gemv_group_direct(a) || (pack_groups && b1::pack_supported(a.act, a.lda, a.M, a.K))))
        return i;
    auto range = [](const void *p, int rows, int64_t ld, int cols, size_t elt, uintptr_t *r0, uintptr_t *r1) {
        *r0 = reinterpret_cast<uintptr_t>(p);
        *r1 = *r0 + ((size_t)(rows - 1) * (size_t)ld + (size_t)cols) * elt;
    };
    uintptr_t in0, in1;
    range(a.act, a.M, a.lda, a.K, sizeof(float), &in0, &in1);
    uintptr_t o0[b1::kGemvGroupMax], o1[b1::kGemvGroupMax];
    int n = 0;
    for (int j = i; j < n_ops && n < b1::kGemvGroupMax; ++j) {
        const BatchOp bj = at(j);
        const bonsai_b1_linear_op &q = *bj.op;
        if (!batch_op_ok(q, bj.epi) || epi_kind(bj.epi) != BONSAI_B1_EPI_NONE || q.batch != a.M ||
            q.act != a.act || q.lda != a.lda || q.w->in_dim != a.K || batch_path(batch_args(q), mode) != BatchPath::Gemv)
            break;
        uintptr_t q0, q1;
        range(q.out, q.batch, q.ldo, q.w->out_dim, sizeof(float), &q0, &q1);
        bool apart = !(q0 < in1 && in0 < q1);
        for (int k = 0; k < n && apart; ++k) apart = !(q0 < o1[k] && o0[k] < q1);
        if (!apart) break;
        ops[n] = b1::GemvGroupOp{static_cast<const uint8_t *>(q.w->data), q.w->out_dim, q.out, q.ldo};
        o0[n] = q0;
        o1[n] = q1;
        ++n;
    }
    if (n < 2 || !b1::gemv_group_ok(a.M, a.K, ops, n)) return i;
    return i + n - 1;
}

// Workspace areas of a batch, laid out [pack][split][y], each 256-byte
// aligned: the largest range-safe packing among its packed GEMMs and
// grouped small-M runs of more than kGemvGroupF32MaxM tokens, the largest split-K partial area among its plain packed GEMMs
// (fused runs included), and the largest fp32 linear output among its ops
// whose epilogue runs as a separate pass (the other paths).
struct BatchAreas {
    size_t pack = 0, split = 0, y = 0;
    size_t split_off() const { return round256(pack); }
    size_t y_off() const { return split_off() + round256(split); }
    size_t need() const { return y ? y_off() + y : split ? split_off() + split : pack; }
};

template <class OpAt>
static BatchAreas batch_areas(int n_ops, int mode, int num_cus, OpAt at, bool pack_groups = true) {
    BatchAreas r;
    for (int i = 0; i < n_ops; ++i) {
        const BatchOp b = at(i);
        if (!batch_op_ok(*b.op, b.epi) || b.op->batch == 0) continue;
        const b1::LinearArgs a = batch_args(*b.op);
        const BatchPath path = batch_path(a, mode);
        if (path == BatchPath::Gemv) {
            b1::GemvGroupOp ops[b1::kGemvGroupMax];
            const int last = gemv_span(n_ops, mode, at, i, ops, pack_groups);
            if (last > i) {
                if (!gemv_group_direct(a)) r.pack = std::max(r.pack, b1::pack_area_bytes(a.M, a.K));
                i = last;
                continue;
            }
        }
        if (path == BatchPath::Packed) r.pack = std::max(r.pack, b1::pack_area_bytes(a.M, a.K));
        if (path == BatchPath::Packed) {
            if (epi_kind(b.epi) == BONSAI_B1_EPI_NONE) {
                int n_sum;
                const int last = fuse_span(n_ops, mode, num_cus, at, i, &n_sum);
                r.split = std::max(r.split,
                                   b1::gemm_split_bytes(a.M, n_sum, b1::gemm_splits(a.M, a.K, a.N, num_cus)));
                i = last;
            }
        } else if (epi_kind(b.epi) != BONSAI_B1_EPI_NONE) {
            r.y = std::max(r.y, (size_t)a.M * (size_t)a.N * sizeof(float));
        }
    }
    return r;
}

template <class OpAt>
static size_t batch_need(int n_ops, int mode, OpAt at) {
    const DeviceInfo *dev = current_device(nullptr);
    return batch_areas(n_ops, mode, dev ? dev->num_cus : 0, at).need();
}

template <class OpAt>
static int batch_run(int n_ops, int mode, int32_t *nonfinite, void *workspace, size_t workspace_bytes, int *bad_op,
                     hipStream_t stream, OpAt at) {
    if (bad_op) *bad_op = -1;
    if (n_ops < 0) return BONSAI_B1_ERR_ARG;
    if (mode < BONSAI_B1_MODE_AUTO || mode > BONSAI_B1_MODE_EXACT) return BONSAI_B1_ERR_ARG;
    for (int i = 0; i < n_ops; ++i) {
        const BatchOp b = at(i);
        int kind;
        b1::GemmEpi g;
        if (!batch_op_ok(*b.op, b.epi) ||
            epi_args(b.epi, b.op->w->out_dim, b.op->batch, b.op->out, b.op->ldo, &kind, &g) != BONSAI_B1_OK) {
            if (bad_op) *bad_op = i;
            return BONSAI_B1_ERR_ARG;
        }
    }
    DeviceInfo *dev = current_device(nullptr);
    if (!dev) return BONSAI_B1_ERR_DEVICE;
    BatchAreas areas = batch_areas(n_ops, mode, dev->num_cus, at);
    WsLease lease;
    bool pack_groups = true;
    if (areas.need() > 0) {
        if (!workspace) {
            lease.acquire(dev, stream, areas.need());
            workspace = lease.ptr();
            workspace_bytes = workspace ? areas.need() : 0;
            if (!workspace) {
                // No library workspace to be had (a capture with no large
                // enough buffer): grouped small-M runs that would read a
                // packing run their ops one by one instead, which needs none.
                const BatchAreas alone = batch_areas(n_ops, mode, dev->num_cus, at, false);
                if (alone.need() == 0) {
                    areas = alone;
                    pack_groups = false;
                }
            }
        }
    }
    if (areas.need() > 0) {
        // a workspace without room for the split-K partials runs every GEMM
        // unsplit (the same outputs up to the order of the K summation)
        if (workspace && workspace_bytes < areas.need()) areas.split = 0;
        if (!workspace || workspace_bytes < areas.need() || (reinterpret_cast<uintptr_t>(workspace) & 15u))
            return BONSAI_B1_ERR_ARG;
        if (!lease.ptr()) {
            // the caller's workspace lies apart from every op's input and
            // outputs (the library's own cannot overlap them)
            const uintptr_t w0 = reinterpret_cast<uintptr_t>(workspace), w1 = w0 + areas.need();
            auto apart = [&](const void *p, int rows, int64_t ld_bytes, int64_t row_bytes) {
                if (!p || rows <= 0 || row_bytes <= 0) return true;
                const uintptr_t p0 = reinterpret_cast<uintptr_t>(p);
                const uintptr_t p1 = p0 + (size_t)(rows - 1) * (size_t)ld_bytes + (size_t)row_bytes;
                return !(p0 < w1 && w0 < p1);
            };
            for (int i = 0; i < n_ops; ++i) {
                const BatchOp b = at(i);
                const bonsai_b1_linear_op &op = *b.op;
                const int kind = epi_kind(b.epi);
                const int n = op.w->out_dim;
                bool ok = apart(op.act, op.batch, op.lda * 4, (int64_t)op.w->in_dim * 4);
                if (kind == BONSAI_B1_EPI_PACKED) {
                    const int split = b.epi->split;
                    const int pcols = b.epi->act == BONSAI_B1_ACT_SWIGLU ? (n - split) / 2 : n - split;
                    ok = ok && apart(op.out, op.batch, op.ldo * 4, (int64_t)split * 4) &&
                         apart(b.epi->packed, op.batch, b.epi->ldp * 2, (int64_t)pcols * 2);
                } else {
                    ok = ok && apart(op.out, op.batch, op.ldo * 4,
                                     (int64_t)(kind == BONSAI_B1_EPI_SWIGLU ? n / 2 : n) * 4);
                }
                if (kind == BONSAI_B1_EPI_GATE_RESIDUAL && b.epi->residual != op.out)
                    ok = ok && apart(b.epi->residual, op.batch, b.epi->ldr * 4, (int64_t)n * 4) &&
                         apart(b.epi->gate, 1, (int64_t)n * 4, (int64_t)n * 4);
                if (!ok) {
                    if (bad_op) *bad_op = i;
                    return BONSAI_B1_ERR_ARG;
                }
            }
        }
    }
    float *ybuf = areas.y ? reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + areas.y_off()) : nullptr;
    void *split_area = areas.split ? static_cast<uint8_t *>(workspace) + areas.split_off() : nullptr;
    // The packed activations in the workspace belong to (act, lda, batch, K).
    const float *packed_act = nullptr;
    int64_t packed_lda = 0;
    int packed_m = 0, packed_k = 0;
    for (int i = 0; i < n_ops; ++i) {
        const BatchOp bo = at(i);
        if (bo.op->batch == 0) continue;
        b1::LinearArgs a = batch_args(*bo.op);
        a.nonfinite = nonfinite;
        int kind;
        b1::GemmEpi g;
        (void)epi_args(bo.epi, a.N, a.M, a.out, a.ldo, &kind, &g);
        int out_cols = kind == BONSAI_B1_EPI_SWIGLU ? a.N / 2 : a.N;
        const BatchPath path = batch_path(a, mode);
        b1::GemvGroupOp gops[b1::kGemvGroupMax];
        const int first = i;
        const int glast = path == BatchPath::Gemv ? gemv_span(n_ops, mode, at, i, gops, pack_groups) : i;
        const bool direct = glast > i && gemv_group_direct(a);
        hipError_t e = hipSuccess;
        // the range-safe packing of this op's input, unless the workspace
        // holds it already
        const float *rsc = nullptr;
        if (path == BatchPath::Packed || (glast > i && !direct)) {
            if (!(packed_act == a.act && packed_lda == a.lda && packed_m == a.M && packed_k == a.K)) {
                e = b1::launch_pack_rows(a.act, a.lda, a.M, a.K, workspace, stream);
                packed_act = a.act;
                packed_lda = a.lda;
                packed_m = a.M;
                packed_k = a.K;
            }
            rsc = b1::pack_area_rsc(workspace, a.M, a.K);
        }
        if (glast > i) {
            // the run's outputs lie apart from its input (gemv_span)
            if (direct)
                e = b1::launch_gemv_group_f32(a.act, a.lda, a.K, a.M, gops, glast - i + 1, nonfinite, dev->num_cus,
                                              stream);
            else if (e == hipSuccess)
                e = b1::launch_gemv_group(workspace, rsc, a.K, a.M, gops, glast - i + 1, nonfinite, dev->num_cus,
                                          stream);
            i = glast;
        } else if (path != BatchPath::Packed) {
            // the linear, into the workspace first when an epilogue follows
            b1::LinearArgs la = a;
            if (kind != BONSAI_B1_EPI_NONE) {
                la.out = ybuf;
                la.ldo = a.N;
            }
            if (e == hipSuccess) {
                switch (path) {
                case BatchPath::Exact: e = b1::launch_exact(la, dev->num_cus, stream); break;
                case BatchPath::Gemv: e = b1::launch_gemv(la, dev->num_cus, stream); break;
                default: e = b1::launch_gemm(la, dev->num_cus, nullptr, 0, stream); break;
                }
            }
            if (e == hipSuccess && kind == BONSAI_B1_EPI_PACKED)
                e = b1::launch_epi_packed(ybuf, a.N, a.M, a.N, g, a.out, a.ldo, stream);
            else if (e == hipSuccess && kind != BONSAI_B1_EPI_NONE)
                e = b1::launch_epi(ybuf, a.N, a.M, a.N, kind, g, a.out, a.ldo, stream);
        } else {
            int n_sum;
            const int last = fuse_span(n_ops, mode, dev->num_cus, at, i, &n_sum);
            const int splits = kind == BONSAI_B1_EPI_NONE ? b1::gemm_splits(a.M, a.K, a.N, dev->num_cus) : 1;
            g.rsc = rsc;
            if (e == hipSuccess) {
                if (splits > 1 && split_area && areas.split >= b1::gemm_split_bytes(a.M, n_sum, splits))
                    e = b1::launch_gemm_packed_split(workspace, a.w, a.K, n_sum, a.M, a.out, a.ldo, nonfinite,
                                                     dev->num_cus, splits, split_area, stream, rsc);
                else
                    e = b1::launch_gemm_packed_epi(workspace, a.w, a.K, n_sum, a.M, a.out, a.ldo, nonfinite,
                                                   dev->num_cus, kind, g, stream);
            }
            if (last > i) out_cols = n_sum;
            i = last;
        }
        if (e != hipSuccess) {
            if (bad_op) *bad_op = i;
            return BONSAI_B1_ERR_HIP;
        }
        // An output written over the packed activations' source invalidates
        // the packing: every output of a grouped small-M run (all its ops
        // share op i's batch), else op i's (or its fused run's) own.
        if (packed_act) {
            const uintptr_t p0 = reinterpret_cast<uintptr_t>(packed_act);
            const uintptr_t p1 = p0 + ((size_t)(packed_m - 1) * (size_t)packed_lda + (size_t)packed_k) * sizeof(float);
            auto hits = [&](const void *o, int64_t ld_bytes, int64_t row_bytes) {
                const uintptr_t o0 = reinterpret_cast<uintptr_t>(o);
                const uintptr_t o1 = o0 + (size_t)(a.M - 1) * (size_t)ld_bytes + (size_t)row_bytes;
                return o0 < p1 && p0 < o1;
            };
            if (glast > first) {
                for (int j = 0; j <= glast - first; ++j)
                    if (hits(gops[j].out, gops[j].ldo * 4, (int64_t)gops[j].N * 4)) packed_act = nullptr;
            } else if (kind == BONSAI_B1_EPI_PACKED) {
                // the fp32 columns and the packed fp16 columns
                const int pcols = g.glu_h ? g.glu_h : a.N - g.split;
                if ((g.split > 0 && hits(a.out, a.ldo * 4, (int64_t)g.split * 4)) ||
                    (pcols > 0 && hits(bo.epi->packed, bo.epi->ldp * 2, (int64_t)pcols * 2)))
                    packed_act = nullptr;
            } else if (hits(a.out, a.ldo * 4, (int64_t)out_cols * 4)) {
                packed_act = nullptr;
            }
        }
    }
    return BONSAI_B1_OK;
}

} // extern "C++"

size_t bonsai_b1_linear_batch_workspace_bytes(const bonsai_b1_linear_op *ops, int n_ops, int mode) {
    if (!ops || n_ops <= 0 || mode < BONSAI_B1_MODE_AUTO || mode > BONSAI_B1_MODE_FAST) return 0;
    return batch_need(n_ops, mode, [&](int i) { return BatchOp{&ops[i], nullptr}; });
}

int bonsai_b1_linear_batch(const bonsai_b1_linear_op *ops, int n_ops, int mode, int32_t *nonfinite,
                           void *workspace, size_t workspace_bytes, int *bad_op, hipStream_t stream) {
    if (n_ops > 0 && !ops) return BONSAI_B1_ERR_ARG;
    return batch_run(n_ops, mode, nonfinite, workspace, workspace_bytes, bad_op, stream,
                     [&](int i) { return BatchOp{&ops[i], nullptr}; });
}

size_t bonsai_b1_linear_batch_epi_workspace_bytes(const bonsai_b1_linear_op_epi *ops, int n_ops, int mode) {
    if (!ops || n_ops <= 0 || mode < BONSAI_B1_MODE_AUTO || mode > BONSAI_B1_MODE_EXACT) return 0;
    return batch_need(n_ops, mode, [&](int i) { return BatchOp{&ops[i].op, &ops[i].epi}; });
}

int bonsai_b1_linear_batch_epi(const bonsai_b1_linear_op_epi *ops, int n_ops, int mode, int32_t *nonfinite,
                               void *workspace, size_t workspace_bytes, int *bad_op, hipStream_t stream) {
    if (n_ops > 0 && !ops) return BONSAI_B1_ERR_ARG;
    return batch_run(n_ops, mode, nonfinite, workspace, workspace_bytes, bad_op, stream,
                     [&](int i) { return BatchOp{&ops[i].op, &ops[i].epi}; });
}

int bonsai_b1_linear(const float *act, const B1Weights *w, int batch,
                     float *out, B1LinearUserData *ud, int mode,
                     int32_t *nonfinite, hipStream_t stream) {
    if (!w) return BONSAI_B1_ERR_ARG;
    if (ud) {
        ud->magic = BONSAI_B1_MAGIC;
        ud->in_dim = w->in_dim;
        ud->out_dim = w->out_dim;
    }
    return bonsai_b1_linear_f32(act, w->in_dim, w->data, w->in_dim, w->out_dim,
                                batch, out, w->out_dim, mode, nonfinite, stream);
}

namespace {
// The callback's non-finite counters, per thread (its ops run on the
// thread's hipStreamPerThread) and device: [0] for per-op checking, [1] the
// deferred count.  Allocated by the thread's first op on a device; they live
// until the process ends.
thread_local bool t_cb_defer = false;
thread_local int32_t *t_cb_count[kMaxDevices][2] = {};
} // namespace

int bonsai_b1_callback_defer(int on) {
    t_cb_defer = on != 0;
    return BONSAI_B1_OK;
}

int bonsai_b1_callback_finish(int32_t *count) {
    int dev = 0;
    if (!current_device(&dev)) return BONSAI_B1_ERR_DEVICE;
    hipStream_t s = hipStreamPerThread;
    int32_t bad = 0;
    int32_t *cnt = t_cb_count[dev][1];
    if (cnt) {
        if (hipMemcpyAsync(&bad, cnt, sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipMemsetAsync(cnt, 0, sizeof(int32_t), s) != hipSuccess)
            return BONSAI_B1_ERR_HIP;
    }
    if (hipStreamSynchronize(s) != hipSuccess) return BONSAI_B1_ERR_HIP;
    if (count) *count = bad;
    return bad ? BONSAI_B1_ERR_NONFINITE : BONSAI_B1_OK;
}

void bonsai_b1_linear_f32_f32(bonsai_b1_tensor *dst, int ith, int nth,
                              void *userdata) {
    (void)nth;
    if (ith != 0) return;
    const B1LinearUserData *ud = static_cast<const B1LinearUserData *>(userdata);
    const bonsai_b1_tensor *act = dst->src[0];
    const bonsai_b1_tensor *wt = dst->src[1];
    if (!ud || ud->magic != BONSAI_B1_MAGIC || !act || !wt || !wt->data) {
        fprintf(stderr, "B1_FATAL: bad custom-op arguments (userdata/src)\n");
        abort();
    }
    const int in_dim = ud->in_dim, out_dim = ud->out_dim;
    const int batch = (int)act->ne[1];
    const int64_t lda = act->nb[1] ? (int64_t)(act->nb[1] / sizeof(float)) : in_dim;
    const int64_t ldo = dst->nb[1] ? (int64_t)(dst->nb[1] / sizeof(float)) : out_dim;
    int dev = 0;
    DeviceInfo *di = current_device(&dev);
    if (!di) {
        fprintf(stderr, "B1_FATAL: no usable gfx950 device\n");
        abort();
    }
    // this thread's counter on this device for the mode in use (threads run
    // their ops on their own streams, so each counts into its own)
    int32_t *&cnt = t_cb_count[dev][t_cb_defer ? 1 : 0];
    if (!cnt && (hipMalloc(reinterpret_cast<void **>(&cnt), sizeof(int32_t)) != hipSuccess ||
                 hipMemset(cnt, 0, sizeof(int32_t)) != hipSuccess)) {
        fprintf(stderr, "B1_FATAL: allocation of the status counter failed\n");
        abort();
    }
    hipStream_t s = hipStreamPerThread;
    if (t_cb_defer) {
        // enqueue only; the non-finite outputs add to the counter
        const int st = bonsai_b1_linear_f32(static_cast<const float *>(act->data), lda, wt->data, in_dim, out_dim,
                                            batch, static_cast<float *>(dst->data), ldo, BONSAI_B1_MODE_AUTO, cnt, s);
        if (st != BONSAI_B1_OK) {
            fprintf(stderr, "B1_FATAL: b1_linear failed: %s (in_dim=%d out_dim=%d)\n",
                    bonsai_b1_status_string(st), in_dim, out_dim);
            abort();
        }
        return;
    }
    int32_t bad = 0;
    // The op in AUTO mode, then, if that made non-finite outputs, again in
    // EXACT mode (the reference's scalar arithmetic): the reference aborts
    // only when its own fp32 sums are non-finite, so a value FAST mode alone
    // cannot represent must not abort here.
    auto run = [&](int mode) {
        int st = hipMemsetAsync(cnt, 0, sizeof(int32_t), s) == hipSuccess ? BONSAI_B1_OK : BONSAI_B1_ERR_HIP;
        if (st == BONSAI_B1_OK)
            st = bonsai_b1_linear_f32(static_cast<const float *>(act->data), lda, wt->data, in_dim, out_dim, batch,
                                      static_cast<float *>(dst->data), ldo, mode, cnt, s);
        if (st == BONSAI_B1_OK &&
            (hipMemcpyAsync(&bad, cnt, sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
             hipStreamSynchronize(s) != hipSuccess))
            st = BONSAI_B1_ERR_HIP;
        return st;
    };
    int st = run(BONSAI_B1_MODE_AUTO);
    if (st == BONSAI_B1_OK && bad) st = run(BONSAI_B1_MODE_EXACT);
    if (st != BONSAI_B1_OK) {
        fprintf(stderr, "B1_FATAL: b1_linear failed: %s (in_dim=%d out_dim=%d)\n",
                bonsai_b1_status_string(st), in_dim, out_dim);
        abort();
    }
    if (bad) {
        fprintf(stderr, "B1_FATAL_OUT: NaN generated in b1_linear! in_dim=%d out_dim=%d (%d non-finite)\n",
                in_dim, out_dim, bad);
        abort();
    }
}

int bonsai_b1_weights_upload(const void *host_packed, size_t nbytes,
                             int in_dim, int out_dim, hipStream_t stream,
                             B1Weights *out) {
    if (!out || !host_packed || in_dim <= 0 || out_dim <= 0 || in_dim % BONSAI_B1_BLOCK_SIZE)
        return BONSAI_B1_ERR_ARG;
    const size_t want = (size_t)out_dim * (size_t)(in_dim / BONSAI_B1_BLOCK_SIZE) * BONSAI_B1_BLOCK_BYTES;
    if (nbytes != want) return BONSAI_B1_ERR_ARG;
    int dev = 0;
    if (!current_device(&dev)) return BONSAI_B1_ERR_DEVICE;
    void *d = nullptr;
    if (hipMalloc(&d, nbytes) != hipSuccess) return BONSAI_B1_ERR_HIP;
    if (hipMemcpyAsync(d, host_packed, nbytes, hipMemcpyHostToDevice, stream) != hipSuccess) {
        (void)hipFree(d);
        return BONSAI_B1_ERR_HIP;
    }
    out->data = d;
    out->in_dim = in_dim;
    out->out_dim = out_dim;
    out->nbytes = nbytes;
    out->device = dev;
    return BONSAI_B1_OK;
}

int bonsai_b1_weights_concat(const B1Weights *parts, int n_parts, hipStream_t stream, B1Weights *out) {
    if (!parts || n_parts <= 0 || !out) return BONSAI_B1_ERR_ARG;
    const int k = parts[0].in_dim;
    size_t total = 0;
    int64_t rows = 0;
    for (int i = 0; i < n_parts; ++i) {
        const B1Weights &p = parts[i];
        if (!p.data || p.in_dim != k || p.out_dim <= 0 ||
            p.nbytes != (size_t)p.out_dim * (size_t)(k / BONSAI_B1_BLOCK_SIZE) * BONSAI_B1_BLOCK_BYTES)
            return BONSAI_B1_ERR_ARG;
        total += p.nbytes;
        rows += p.out_dim;
    }
    if (k <= 0 || k % BONSAI_B1_BLOCK_SIZE || rows > INT32_MAX) return BONSAI_B1_ERR_ARG;
    int dev = 0;
    if (!current_device(&dev)) return BONSAI_B1_ERR_DEVICE;
    void *d = nullptr;
    if (hipMalloc(&d, total) != hipSuccess) return BONSAI_B1_ERR_HIP;
    size_t off = 0;
    for (int i = 0; i < n_parts; ++i) {
        if (hipMemcpyAsync(static_cast<uint8_t *>(d) + off, parts[i].data, parts[i].nbytes, hipMemcpyDeviceToDevice,
                           stream) != hipSuccess) {
            (void)hipStreamSynchronize(stream);
            (void)hipFree(d);
            return BONSAI_B1_ERR_HIP;
        }
        off += parts[i].nbytes;
    }
    out->data = d;
    out->in_dim = k;
    out->out_dim = (int)rows;
    out->nbytes = total;
    out->device = dev;
    return BONSAI_B1_OK;
}

int bonsai_b1_weights_free(B1Weights *w) {
    if (!w) return BONSAI_B1_ERR_ARG;
    if (w->data) {
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess) return BONSAI_B1_ERR_HIP;
        if (cur != w->device && hipSetDevice(w->device) != hipSuccess) return BONSAI_B1_ERR_HIP;
        hipError_t e = hipFree(w->data);
        if (cur != w->device) (void)hipSetDevice(cur);
        if (e != hipSuccess) return BONSAI_B1_ERR_HIP;
    }
    w->data = nullptr;
    w->nbytes = 0;
    return BONSAI_B1_OK;
}

} // extern "C"
