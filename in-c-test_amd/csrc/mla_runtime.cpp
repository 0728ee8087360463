// Host runtime of libkvl_mla: the reference MLA C API (include/kvl/ops.h, mla_state.h,
// mla_compressed_state.h, mla_compressed_q8_state.h) re-implemented over HIP on one MI355X,
// plus the extensions of include/kvl/mla_hip.h.
//
// Contract kept from the reference (src/mla_compressed_q8_state.c, mla_compressed_state.c,
// mla_state.c): states own calloc'd host arrays that stay authoritative; every call is
// synchronous with host buffers; -1 on invalid arguments with the state unchanged; weights
// are borrowed per call. What the GPU adds:
//   * a device mirror per state (keyed by the struct address, validated against its host
//     pointers and capacity) with a watermark of rows already on the device. Appended rows
//     are produced on the device and written back to the host arrays; rows the caller adds
//     on the host (len above the watermark) are uploaded before use; truncate/reset lower
//     the watermark; *_sync forces a full re-upload.
//   * a device weight cache keyed by host address + size + sampled digest, or pinned by
//     kvl_mla_bind_weights.
//   * one HIP stream; kernels are enqueued in order, results copied back, then synchronised.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "kvl/mla_compressed_q8_state.h"
#include "kvl/mla_compressed_state.h"
#include "kvl/mla_hip.h"
#include "kvl/mla_state.h"
#include "kvl/ops.h"
#include "mla_internal.h"

using namespace kvl;

// Device scratch of the no-allocation decode entry point
// (kvl_mla_decode_compressed_q8_batch_device_noalloc): the decode workspace of up to
// kNoAllocMaxBatch sequences followed by the split-K partials. Every GPU the library runs on
// holds its own copy for the life of the process. Host code never uses the array's name as a
// device address: its address on each device comes from hipGetSymbolAddress at set-up.
constexpr size_t kNoAllocScratchBytes = (size_t)24 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kNoAllocMaxBatch = 16;
constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices];  // device address of `scratch` per device (null: not resolved)

thread_local std::string g_err;

void set_err(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}

#define HIP_TRY(expr)                                                                   \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess) {                                                         \
            set_err("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__,   \
                    __LINE__);                                                          \
            return -1;                                                                  \
        }                                                                               \
    } while (0)

// ---------------------------------------------------------------- device buffers --------

struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
};

// hipFree of library-owned device memory (see Ctx::free_gen).
hipError_t dev_free(void *p);

int dev_reserve(DevBuf &b, size_t bytes) {
    if (bytes <= b.bytes) return 0;
    if (b.p) {
        hipError_t e = dev_free(b.p);
        b.p = nullptr;
        b.bytes = 0;
        if (e != hipSuccess) {
            set_err("hipFree: %s", hipGetErrorString(e));
            return -1;
        }
    }
    size_t want = bytes < 4096 ? 4096 : bytes + bytes / 4;
    hipError_t e = hipMalloc(&b.p, want);
    if (e != hipSuccess) {
        b.p = nullptr;
        set_err("hipMalloc(%zu): %s", want, hipGetErrorString(e));
        return -1;
    }
    b.bytes = want;
    return 0;
}

struct PinBuf {
    void *p = nullptr;
    size_t bytes = 0;
};

int pin_reserve(PinBuf &b, size_t bytes) {
    if (bytes <= b.bytes) return 0;
    if (b.p) (void)hipHostFree(b.p);
    b.p = nullptr;
    b.bytes = 0;
    size_t want = bytes < 65536 ? 65536 : bytes + bytes / 4;
    hipError_t e = hipHostMalloc(&b.p, want, hipHostMallocDefault);
    if (e != hipSuccess) {
        b.p = nullptr;
        set_err("hipHostMalloc(%zu): %s", want, hipGetErrorString(e));
        return -1;
    }
    b.bytes = want;
    return 0;
}

// ---------------------------------------------------------------- context ---------------

struct WeightEntry {
    size_t bytes = 0;
    uint64_t digest = 0;
    void *dev = nullptr;
    void *dev16 = nullptr;  // fp16 copy (prefill o_proj) times 2^f16_shift, valid when f16_ok
    bool f16_ok = false;
    int f16_shift = 0;
    float row_l2max = -1.0f;  // kv_b: max L2 norm of the V rows (prefill V scale); < 0: not yet
    void *devt = nullptr;   // W_UK^T of a kv_b array (decode query preparation), valid when t_ok
    bool t_ok = false;
    int pins = 0;
};

struct Mirror {
    int fmt = 0;
    const void *ha = nullptr, *hb = nullptr, *hc = nullptr;  // host arrays at creation
    int capacity = 0;
    int d0 = 0, d1 = 0, d2 = 0;  // Q8/F32: R, DR; Exp: NH, QD, DV
    void *a = nullptr, *b = nullptr, *c = nullptr;
    int synced = 0;  // rows [0, synced) valid on the device
};

struct RopeTable {
    float2 *dev = nullptr;
    int npos = 0;
};

struct Ctx {
    std::recursive_mutex mu;
    bool ready = false;
    int device = 0;
    int ncu = 256;
    hipStream_t stream = nullptr;
    std::unordered_map<const void *, WeightEntry> weights;
    std::unordered_map<const void *, Mirror> mirrors;
    std::unordered_map<uint64_t, RopeTable> ropes;  // key: theta bits << 16 | DR
    DevBuf work, part, scores, prefill, fill, fillx, layer, sink;
    DevBuf rflag;  // int: raised by a stream-ordered prefill outside the MFMA route's range
    PinBuf pin_in, pin_out;
    // fused Q8 decode (the attention launch prepares the queries and appends the rows, and where
    // the shapes allow also computes the q_proj | kv_a projection and combines the splits): its
    // readiness flags and counters (device, kFqFlagLines lines; cleared by the o_proj launch
    // after each fused launch, or by the separate q_proj | kv_a launch before it) and a
    // host-visible word raised if one of its waits timed out
    unsigned *fq_flags = nullptr;
    int *fq_err = nullptr;
    bool fq_on = true;    // KVL_MLA_NO_FUSED_QPREP=1 turns the fused form off (the two-launch form)
    bool comb_on = true;  // KVL_MLA_NO_FUSED_COMBINE=1: the fused form keeps the combine launch
    bool gemv_on = true;  // KVL_MLA_NO_FUSED_PROJECTION=1: the fused form keeps the projection launch
    unsigned fq_spin = kFqSpinTicks;  // bound of the fused form's device waits (kvl_mla_set_fused_wait_limit)
    // a fused attention launch was enqueued and the o_proj launch that clears its flags was not
    // (an error in between): the next launch that relies on clean flags clears them first
    bool fq_dirty = false;
    bool capturing = false;
    // bumped by every release of library-owned device memory: a graph captured before a bump
    // may hold pointers to freed memory (kvl_mla_graph_launch refuses it)
    uint64_t free_gen = 0;
    // per-stage event timing of decode steps (kvl_mla_timing_*)
    bool timing = false;
    bool timing_graph = false;  // also record into a graph being captured (event-record nodes)
    unsigned timing_mask = (1u << 6) - 1;  // stages bracketed (bit i: stage i)
    std::vector<hipEvent_t> ev_pool;
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> ev_used;
};

constexpr int kStages = 6;  // gemv_in, append, qprep, attention, combine, gemv_out

Ctx &ctx() {
    static Ctx *c = new Ctx();  // never destroyed: device memory is released by the driver
    return *c;
}

// Frees library memory after the work queued on the library stream (which may still read it)
// has finished.
hipError_t dev_free(void *p) {
    Ctx &c = ctx();
    ++c.free_gen;
    if (c.stream && !c.capturing) {
        const hipError_t e = hipStreamSynchronize(c.stream);
        if (e != hipSuccess) return e;
    }
    return hipFree(p);
}

int ensure_ready() {
    Ctx &c = ctx();
    if (c.ready) return 0;
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err("libkvl_mla is built for gfx950; device %d is %s", dev, prop.gcnArchName);
        return -1;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_err("device index %d out of range", dev);
        return -1;
    }
    if (!g_scratch[dev]) {
        void *p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch[dev] = p;
    }
    HIP_TRY(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    HIP_TRY(hipMalloc(&c.fq_flags, kFqFlagLines * kFqFlagStride * sizeof(unsigned)));
    HIP_TRY(hipMemset(c.fq_flags, 0, kFqFlagLines * kFqFlagStride * sizeof(unsigned)));
    HIP_TRY(hipHostMalloc((void **)&c.fq_err, sizeof(int), hipHostMallocDefault));
    *c.fq_err = 0;
    {
        const char *e = getenv("KVL_MLA_NO_FUSED_QPREP");
        c.fq_on = !(e && e[0] == '1');
        e = getenv("KVL_MLA_NO_FUSED_COMBINE");
        c.comb_on = !(e && e[0] == '1');
        e = getenv("KVL_MLA_NO_FUSED_PROJECTION");
        c.gemv_on = !(e && e[0] == '1');
    }
    c.device = dev;
    c.ncu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    c.ready = true;
    return 0;
}

hipEvent_t ev_get() {
    Ctx &c = ctx();
    if (!c.ev_pool.empty()) {
        hipEvent_t e = c.ev_pool.back();
        c.ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Brackets one launch of stage `st` with events when timing is on (during capture only in
// timing mode 2, as event-record nodes of the graph).
struct StageTimer {
    int stage;
    hipEvent_t a = nullptr, b = nullptr;
    explicit StageTimer(int s) : stage(s) {
        Ctx &c = ctx();
        if (s < 0 || !c.timing || !((c.timing_mask >> s) & 1u) || (c.capturing && !c.timing_graph)) return;  // s < 0: not timed
        a = ev_get();
        b = ev_get();
        // inside a capture, only an external record becomes a timestamped node of the graph
        if (a && b) (void)hipEventRecordWithFlags(a, c.stream, c.capturing ? hipEventRecordExternal : 0);
    }
    ~StageTimer() {
        Ctx &c = ctx();
        if (!a || !b) return;
        (void)hipEventRecordWithFlags(b, c.stream, c.capturing ? hipEventRecordExternal : 0);
        c.ev_used.push_back({stage, {a, b}});
    }
};

// ---------------------------------------------------------------- shapes ----------------

bool dims_of(const KvlMlaConfig *cfg, Dims &d) {
    if (!cfg || cfg->hidden_size <= 0 || cfg->num_heads <= 0 || cfg->qk_nope_dim <= 0 ||
        cfg->qk_rope_dim <= 0 || (cfg->qk_rope_dim & 1) || cfg->v_head_dim <= 0 ||
        cfg->kv_lora_rank <= 0 || cfg->rope_theta <= 0.0f)
        return false;
    d.H = cfg->hidden_size;
    d.NH = cfg->num_heads;
    d.DN = cfg->qk_nope_dim;
    d.DR = cfg->qk_rope_dim;
    d.DV = cfg->v_head_dim;
    d.R = cfg->kv_lora_rank;
    d.QD = d.DN + d.DR;
    d.QO = d.NH * d.QD;
    d.KVO = d.R + d.DR;
    d.KVB = d.NH * (d.DN + d.DV);
    d.HO = d.NH * d.DV;
    return true;
}

// Kernel bounds of the device path (kMaxR / kMaxDR / kMaxDN in mla_decode.hip).
bool dims_supported(const Dims &d) {
    if (d.R > 1024 || d.DR > 256 || d.DN > 512) {
        set_err("dims beyond the device kernels' bounds (R<=1024, DR<=256, DN<=512)");
        return false;
    }
    return true;
}

bool kimi_attn(const Dims &d) { return d.NH == 16 && d.R == 512 && d.DR == 64; }

// ---------------------------------------------------------------- weights ---------------

// Word-wise digest state: four independent multiply-xorshift lanes, so the sampled words are
// mixed in parallel (a byte-serial hash of the 5.8 KB that the five weight arrays' samples
// hold cost ≈ 5 µs per host call; this takes well under one).
struct Digest {
    uint64_t v[4] = {0x243f6a8885a308d3ull, 0x13198a2e03707344ull, 0xa4093822299f31d0ull, 0x082efa98ec4e6c89ull};
    static uint64_t mix(uint64_t h, uint64_t w) {
        h = (h ^ w) * 0x9e3779b97f4a7c15ull;
        return h ^ (h >> 29);
    }
    // bytes [p, p + n): whole 32-byte groups over the four lanes, then the tail bytes
    void add(const void *p, size_t n) {
        const unsigned char *b = (const unsigned char *)p;
        size_t i = 0;
        for (; i + 32 <= n; i += 32)
            for (int k = 0; k < 4; ++k) {
                uint64_t w;
                memcpy(&w, b + i + 8 * k, 8);
                v[k] = mix(v[k], w);
            }
        for (int k = 0; i < n; ++i, k = (k + 1) & 3) v[k] = mix(v[k], b[i]);
    }
    uint64_t value() const { return mix(mix(v[0], v[1]), mix(v[2], v[3])); }
};

// Digest of 18 sampled 64-byte windows (first, last and 16 evenly spaced) plus the size.
uint64_t sample_digest(const void *p, size_t bytes) {
    Digest h;
    h.add(&bytes, sizeof bytes);
    const unsigned char *b = (const unsigned char *)p;
    const size_t win = 64;
    if (bytes <= 18 * win) {
        h.add(b, bytes);
        return h.value();
    }
    h.add(b, win);
    h.add(b + bytes - win, win);
    for (int i = 1; i <= 16; ++i) {
        const size_t off = (bytes - win) / 17 * (size_t)i;
        h.add(b + off, win);
    }
    return h.value();
}

int dev_weight(const uint16_t *host, size_t elems, const uint16_t **out) {
    Ctx &c = ctx();
    const size_t bytes = elems * sizeof(uint16_t);
    auto it = c.weights.find(host);
    if (it != c.weights.end() && it->second.bytes == bytes) {
        if (it->second.pins > 0 || it->second.digest == sample_digest(host, bytes)) {
            *out = (const uint16_t *)it->second.dev;
            return 0;
        }
    }
    if (c.capturing) {
        set_err("weight upload during graph capture (bind the weights or run one call first)");
        return -1;
    }
    WeightEntry e;
    if (it != c.weights.end()) {
        e = it->second;
        if (e.bytes != bytes) {
            HIP_TRY(dev_free(e.dev));
            e.dev = nullptr;
        }
    }
    if (!e.dev) HIP_TRY(hipMalloc(&e.dev, bytes));
    if (e.dev16 && e.bytes != bytes) {
        HIP_TRY(dev_free(e.dev16));
        e.dev16 = nullptr;
    }
    if (e.devt && e.bytes != bytes) {
        HIP_TRY(dev_free(e.devt));
        e.devt = nullptr;
    }
    e.bytes = bytes;
    e.f16_ok = false;
    e.t_ok = false;
    e.row_l2max = -1.0f;
    // The blocking copy runs on the null stream, which does not wait for the library's
    // non-blocking stream: when it overwrites a buffer that queued kernels may still read (an
    // unbound array rewritten in place and used again by a stream-ordered device call), finish
    // that work first.
    if (it != c.weights.end()) HIP_TRY(hipStreamSynchronize(c.stream));
    HIP_TRY(hipMemcpy(e.dev, host, bytes, hipMemcpyHostToDevice));
    e.digest = sample_digest(host, bytes);
    c.weights[host] = e;
    *out = (const uint16_t *)e.dev;
    return 0;
}

float bf16_abs(uint16_t b) {
    const uint32_t u = (uint32_t)(b & 0x7fff) << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

// fp16 copy of a weight array times 2^shift (converted on the device from its bf16 copy,
// stream-ordered). shift puts the largest |w| in [2^13, 2^14): far from the fp16 maximum
// (65504) and with the array's small values above the fp16 subnormals as far as the bf16
// values allow; a power of two, so the conversion stays exact and the product's scale is
// undone exactly.
int dev_weight_f16(const uint16_t *host, size_t elems, const _Float16 **out, int *shift) {
    Ctx &c = ctx();
    const uint16_t *d16;
    if (dev_weight(host, elems, &d16) != 0) return -1;
    WeightEntry &e = c.weights[host];
    if (!e.f16_ok) {
        if (c.capturing) {
            set_err("fp16 weight conversion during graph capture");
            return -1;
        }
        float mx = 0.f;
        for (size_t i = 0; i < elems; ++i) mx = std::max(mx, bf16_abs(host[i]));
        int ex = 0;
        e.f16_shift = 0;
        if (mx > 0.f && std::isfinite(mx)) {
            (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
            e.f16_shift = std::min(100, std::max(-100, 14 - ex));
        }
        if (!e.dev16) HIP_TRY(hipMalloc(&e.dev16, e.bytes));
        HIP_TRY(launch_bf16_to_f16(c.stream, (_Float16 *)e.dev16, d16, elems, ldexpf(1.0f, e.f16_shift)));
        e.f16_ok = true;
    }
    *out = (const _Float16 *)e.dev16;
    *shift = e.f16_shift;
    return 0;
}

// Power-of-two scale for the prefill's V (and attention output) in fp16: from the bound
// |v| = |kv_b_row . latent| <= ||kv_b_row||_2 ||latent||_2 with ||latent||_2 <= sqrt(R)
// max|kv_a_norm| (an RMSNorm output has ||x / rms(x)||_2 <= sqrt(R)), the scale puts the
// bound below 2^14 (the fp16 maximum is 65504).
float prefill_vscale(const KvlMlaBF16 *w, const Dims &d) {
    Ctx &c = ctx();
    auto it = c.weights.find(w->kv_b_proj);
    if (it == c.weights.end()) return 1.0f;
    WeightEntry &e = it->second;
    if (e.row_l2max < 0.f) {
        double mx = 0.0;
        for (int h = 0; h < d.NH; ++h)
            for (int r = 0; r < d.DV; ++r) {
                const uint16_t *row = w->kv_b_proj + ((size_t)h * (d.DN + d.DV) + d.DN + r) * d.R;
                double ss = 0.0;
                for (int k = 0; k < d.R; ++k) {
                    const double v = bf16_abs(row[k]);
                    ss += v * v;
                }
                mx = std::max(mx, sqrt(ss));
            }
        e.row_l2max = (float)mx;
    }
    float nmax = 0.f;
    for (int k = 0; k < d.R; ++k) nmax = std::max(nmax, bf16_abs(w->kv_a_norm[k]));
    const double bound = 1.001 * sqrt((double)d.R) * (double)nmax * (double)e.row_l2max;
    if (!(bound > 0.0) || !std::isfinite(bound)) return 1.0f;
    int ex = 0;
    (void)frexp(bound, &ex);  // bound < 2^ex
    return ldexpf(1.0f, std::min(100, std::max(-100, 14 - ex)));
}

// W_UK^T of a kv_b array in MFMA fragment order (transposed on the device from its bf16 copy,
// stream-ordered): the A operands of the decode's query preparation for the Kimi shapes.
bool ukt_shape(const Dims &d) { return d.R == 512 && d.DN == 128; }

int dev_weight_ukt(const uint16_t *host, const Dims &d, const uint16_t **out) {
    Ctx &c = ctx();
    const uint16_t *kvb;
    if (dev_weight(host, (size_t)d.KVB * d.R, &kvb) != 0) return -1;
    WeightEntry &e = c.weights[host];
    if (!e.t_ok) {
        if (c.capturing) {
            set_err("W_UK transpose during graph capture (bind the weights or run one call first)");
            return -1;
        }
        if (!e.devt) HIP_TRY(hipMalloc(&e.devt, (size_t)d.NH * d.R * d.DN * sizeof(uint16_t)));
        HIP_TRY(launch_wuk_transpose(c.stream, (uint16_t *)e.devt, kvb, d));
        e.t_ok = true;
    }
    *out = (const uint16_t *)e.devt;
    return 0;
}

struct DevWeights {
    const uint16_t *q, *kva, *norm, *kvb, *o;
    const uint16_t *ukt = nullptr;  // W_UK^T (Kimi shapes), else null
};

int dev_weights(const KvlMlaBF16 *w, const Dims &d, DevWeights &dw) {
    if (dev_weight(w->q_proj, (size_t)d.QO * d.H, &dw.q) != 0) return -1;
    if (dev_weight(w->kv_a_proj, (size_t)d.KVO * d.H, &dw.kva) != 0) return -1;
    if (dev_weight(w->kv_a_norm, (size_t)d.R, &dw.norm) != 0) return -1;
    if (dev_weight(w->kv_b_proj, (size_t)d.KVB * d.R, &dw.kvb) != 0) return -1;
    if (dev_weight(w->o_proj, (size_t)d.H * d.HO, &dw.o) != 0) return -1;
    dw.ukt = nullptr;
    if (ukt_shape(d) && dev_weight_ukt(w->kv_b_proj, d, &dw.ukt) != 0) return -1;
    return 0;
}

bool weights_ok(const KvlMlaBF16 *w) {
    return w && w->q_proj && w->kv_a_proj && w->kv_a_norm && w->kv_b_proj && w->o_proj;
}

// ---------------------------------------------------------------- RoPE table ------------

uint64_t rope_key(float theta, int DR) {
    uint32_t tb;
    memcpy(&tb, &theta, sizeof tb);
    return ((uint64_t)tb << 16) | (uint64_t)DR;
}

// The existing table when it covers positions [0, need_pos), without growing it.
int rope_lookup(float theta, int DR, int need_pos, const float2 **out) {
    Ctx &c = ctx();
    auto it = c.ropes.find(rope_key(theta, DR));
    if (it == c.ropes.end() || it->second.npos < need_pos) {
        set_err("the RoPE table does not cover position %d yet (a decode at that position or later "
                "through an allocating entry point builds it)", need_pos - 1);
        return -1;
    }
    *out = it->second.dev;
    return 0;
}

// (cos, sin) of pos * theta^(-2i/DR) computed exactly as src/mla_compressed_q8_state.c:22-25:
// double pow/cos/sin, rounded to float. The device kernels only apply the rotation.
int rope_table(float theta, int DR, int need_pos, const float2 **out) {
    Ctx &c = ctx();
    RopeTable &t = c.ropes[rope_key(theta, DR)];
    if (need_pos > t.npos) {
        if (c.capturing) {
            set_err("RoPE table growth during graph capture");
            return -1;
        }
        int npos = 1024;
        while (npos < need_pos) npos *= 2;
        const int half = DR / 2;
        std::vector<float2> h((size_t)npos * half);
        for (int i = 0; i < half; ++i) {
            const double freq = pow((double)theta, -((double)(2 * i) / (double)DR));
            for (int p = 0; p < npos; ++p) {
                const double ang = (double)p * freq;
                h[(size_t)p * half + i] = make_float2((float)cos(ang), (float)sin(ang));
            }
        }
        if (t.dev) HIP_TRY(dev_free(t.dev));
        t.dev = nullptr;
        t.npos = 0;
        HIP_TRY(hipMalloc((void **)&t.dev, h.size() * sizeof(float2)));
        HIP_TRY(hipMemcpy(t.dev, h.data(), h.size() * sizeof(float2), hipMemcpyHostToDevice));
        t.npos = npos;
    }
    *out = t.dev;
    return 0;
}

// ---------------------------------------------------------------- state mirrors ---------

size_t row_bytes_of(int fmt, int d0, int d1, int d2) {
    if (fmt == kFmtQ8) return (size_t)d0 + 4 + 2 * (size_t)d1;
    if (fmt == kFmtF32) return 4 * ((size_t)d0 + (size_t)d1);
    if (fmt == kFmtBF16) return 2 * ((size_t)d0 + (size_t)d1);
    return 4 * (size_t)d0 * ((size_t)d1 + (size_t)d2);
}

void mirror_free(Mirror &m) {
    if (m.a) (void)dev_free(m.a);
    if (m.b) (void)dev_free(m.b);
    if (m.c) (void)dev_free(m.c);
    m.a = m.b = m.c = nullptr;
}

void mirror_drop(const void *key) {
    Ctx &c = ctx();
    auto it = c.mirrors.find(key);
    if (it == c.mirrors.end()) return;
    mirror_free(it->second);
    c.mirrors.erase(it);
}

void mirror_lower(const void *key, int len) {
    Ctx &c = ctx();
    auto it = c.mirrors.find(key);
    if (it != c.mirrors.end() && it->second.synced > len) it->second.synced = len;
}

// Host array sizes (elements) of each component per row.
struct HostView {
    int fmt;
    const void *ha, *hb, *hc;
    int capacity, len;
    int d0, d1, d2;
};

HostView view_of(const KvlMlaCompressedQ8State *s) {
    return {kFmtQ8, s->latent_q8, s->latent_scale, s->rope_bf16, s->capacity, s->len,
            s->kv_lora_rank, s->qk_rope_dim, 0};
}
HostView view_of(const KvlMlaCompressedState *s) {
    return {kFmtF32, s->latent, s->rope, nullptr, s->capacity, s->len, s->kv_lora_rank,
            s->qk_rope_dim, 0};
}
HostView view_of(const KvlMlaCompressedBF16State *s) {
    return {kFmtBF16, s->latent, s->rope, nullptr, s->capacity, s->len, s->kv_lora_rank,
            s->qk_rope_dim, 0};
}
HostView view_of(const KvlMlaState *s) {
    return {kFmtExp, s->keys, s->values, nullptr, s->capacity, s->len, s->num_heads,
            s->qk_nope_dim + s->qk_rope_dim, s->v_head_dim};
}

// Element sizes (bytes) of the arrays a/b/c per row.
void comp_bytes(int fmt, int d0, int d1, int d2, size_t &ea, size_t &eb, size_t &ec) {
    if (fmt == kFmtQ8) {
        ea = (size_t)d0;
        eb = 4;
        ec = 2 * (size_t)d1;
    } else if (fmt == kFmtF32) {
        ea = 4 * (size_t)d0;
        eb = 4 * (size_t)d1;
        ec = 0;
    } else if (fmt == kFmtBF16) {
        ea = 2 * (size_t)d0;
        eb = 2 * (size_t)d1;
        ec = 0;
    } else {
        ea = 4 * (size_t)d0 * d1;
        eb = 4 * (size_t)d0 * d2;
        ec = 0;
    }
}

int upload_rows(Mirror &m, const HostView &v, int r0, int r1, hipStream_t st) {
    if (r1 <= r0) return 0;
    size_t ea, eb, ec;
    comp_bytes(m.fmt, m.d0, m.d1, m.d2, ea, eb, ec);
    const size_t n = (size_t)(r1 - r0);
    HIP_TRY(hipMemcpyAsync((char *)m.a + ea * r0, (const char *)v.ha + ea * r0, ea * n,
                           hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync((char *)m.b + eb * r0, (const char *)v.hb + eb * r0, eb * n,
                           hipMemcpyHostToDevice, st));
    if (ec)
        HIP_TRY(hipMemcpyAsync((char *)m.c + ec * r0, (const char *)v.hc + ec * r0, ec * n,
                               hipMemcpyHostToDevice, st));
    return 0;
}

// Device mirror of a state, created or re-created when the host arrays changed, and synced
// up to the host len (unless `no_upload`, used by the synthetic fill).
int mirror_get(const void *key, const HostView &v, Mirror **out, bool no_upload = false) {
    Ctx &c = ctx();
    auto it = c.mirrors.find(key);
    if (it != c.mirrors.end()) {
        Mirror &m = it->second;
        if (m.fmt != v.fmt || m.ha != v.ha || m.hb != v.hb || m.hc != v.hc ||
            m.capacity != v.capacity || m.d0 != v.d0 || m.d1 != v.d1 || m.d2 != v.d2) {
            mirror_free(m);
            c.mirrors.erase(it);
            it = c.mirrors.end();
        }
    }
    if (it == c.mirrors.end()) {
        if (c.capturing) {
            set_err("state mirror creation during graph capture");
            return -1;
        }
        Mirror m;
        m.fmt = v.fmt;
        m.ha = v.ha;
        m.hb = v.hb;
        m.hc = v.hc;
        m.capacity = v.capacity;
        m.d0 = v.d0;
        m.d1 = v.d1;
        m.d2 = v.d2;
        size_t ea, eb, ec;
        comp_bytes(v.fmt, v.d0, v.d1, v.d2, ea, eb, ec);
        const size_t cap = (size_t)v.capacity;
        hipError_t e = hipMalloc(&m.a, ea * cap);
        if (e == hipSuccess) e = hipMalloc(&m.b, eb * cap);
        if (e == hipSuccess && ec) e = hipMalloc(&m.c, ec * cap);
        if (e != hipSuccess) {
            mirror_free(m);
            set_err("state mirror allocation (%zu rows): %s", cap, hipGetErrorString(e));
            return -1;
        }
        it = c.mirrors.emplace(key, m).first;
    }
    Mirror &m = it->second;
    if (m.synced > v.len) m.synced = v.len;
    if (!no_upload && m.synced < v.len) {
        if (upload_rows(m, v, m.synced, v.len, c.stream) != 0) return -1;
        m.synced = v.len;
    }
    *out = &m;
    return 0;
}

// ---------------------------------------------------------------- workspace -------------

struct Layout {
    size_t off = 0;
    template <class T>
    T *take(char *base, size_t n) {
        off = (off + 255) & ~(size_t)255;
        T *p = (T *)(base + off);
        off += n * sizeof(T);
        return p;
    }
};

// Carves DecodeWork for a group of B sequences out of `base` (nullptr: sizing only); returns
// the bytes it spans.
size_t decode_work_at(const Dims &d, int B, int row_bytes, char *base, DecodeWork &w) {
    const size_t qs = (size_t)std::max(d.R + d.DR, d.QD);
    auto carve = [&](char *base, Layout &L) {
        w.x = L.take<float>(base, (size_t)B * d.H);
        w.y = L.take<float>(base, (size_t)kGemvKs * B * (d.QO + d.KVO));  // room for the partials
        w.ynp = 1;
        w.ypstride = 0;
        w.qf = L.take<float>(base, (size_t)B * d.NH * qs);
        w.qhi = L.take<int8_t>(base, (size_t)B * d.NH * d.R);
        w.qlo = L.take<int8_t>(base, (size_t)B * d.NH * d.R);
        w.qs = L.take<float>(base, (size_t)B * d.NH);
        w.qrhi = L.take<uint16_t>(base, (size_t)B * d.NH * d.DR);
        w.qrlo = L.take<uint16_t>(base, (size_t)B * d.NH * d.DR);
        w.latent = L.take<float>(base, (size_t)B * d.R);
        w.kv = L.take<float>(base, (size_t)B * d.KVB);
        w.mix = L.take<float>(base, (size_t)B * d.NH * std::max(d.R, d.DV));
        w.ho = L.take<float>(base, (size_t)B * d.HO);
        w.hos = L.take<uint16_t>(base, (size_t)2 * B * d.HO);
        w.out = L.take<float>(base, (size_t)B * d.H);
        w.rows = L.take<uint8_t>(base, (size_t)B * row_bytes);
    };
    Layout L;
    carve(base, L);
    w.part = nullptr;
    return (L.off + 255) & ~(size_t)255;
}

// DecodeWork for a group of B sequences in the library's workspace buffer (grown on demand).
int decode_work(const Dims &d, int B, int row_bytes, DecodeWork &w) {
    Ctx &c = ctx();
    const size_t need = decode_work_at(d, B, row_bytes, nullptr, w);
    if (c.work.bytes < need) {
        if (c.capturing) {
            set_err("workspace growth during graph capture");
            return -1;
        }
        if (dev_reserve(c.work, need) != 0) return -1;
    }
    decode_work_at(d, B, row_bytes, (char *)c.work.p, w);
    return 0;
}

int reserve_part(size_t bytes, float **p) {
    Ctx &c = ctx();
    if (c.part.bytes < bytes) {
        if (c.capturing) {
            set_err("partials growth during graph capture");
            return -1;
        }
        if (dev_reserve(c.part, bytes) != 0) return -1;
    }
    *p = (float *)c.part.p;
    return 0;
}

// ---------------------------------------------------------------- decode core -----------

struct SeqIn {
    Mirror *m;
    int pos;
};

// Split-K plan of the MFMA attention kernels. The kernels run about wg_per_cu workgroups per CU
// (one for the Q8 kernel, whose LDS ring fills a CU; two for the BF16 and FP32 kernels, whose
// two-slot rings take half of it), so a launch should have at most that many splits: one more
// makes a second round of workgroups that doubles the launch time.
int plan_chunk(int kind) { return kind == kAttnQ8Mfma ? 64 : kind == kAttnBF16Mfma ? 32 : 16; }
int plan_wg_per_cu(int kind) {
    return kind == kAttnQ8Mfma ? 1 : kind == kAttnF32Mfma || kind == kAttnBF16Mfma ? 2 : 3;
}

// Splits of a history of len rows at r rows per split. Q8: a remainder of at most r/8 rows past
// the last full split joins that split (its 1024-row cap would otherwise leave a one-row split
// past the CU count, e.g. 8 x 32769 rows); the other kinds: ceil(len / r).
long nsplit_of(int kind, long len, long r) {
    if (kind == kAttnQ8Mfma) return std::max(1L, (len + r - 1 - r / 8) / r);
    return std::max(1L, (len + r - 1) / r);
}

// Rows per split shared by the sequences of a launch: the smallest multiple of the kernel's chunk
// (at least four chunks) whose split count sum_i nsplit_of(len_i, r) fits wg_per_cu x ncu, so the
// launch runs as one round of workgroups. Q8: at most 1024 rows (long batches then take more
// than one round). A lone sequence gets splits of at least two chunks, at most lone_splits(kind,
// len) of them: its launch is bound by the workgroups' fixed start-up (about 11 us with one or
// two chunks each) and the combine, whose partials grow with the split count (measured, one
// decode over 8K / 32K Q8 rows, attention + combine: 19.3 / 31.3 us with 32 splits of >= 4
// chunks, 17.5 / 23.7 us with 64 of >= 2, 20.7 / 23.7 us with 128 of >= 1). The lone plan is also
// the plan of each token of a block decode (bit-identical to single decodes): with 64 splits at
// 32K Q8 rows the 64 x 8 workgroups of an 8-token block take two rounds (host calls: single
// 0.063 -> 0.057 ms, 8-token block 0.077 -> 0.085 ms, 1.49x the single decode).
long lone_splits(int kind, long len) {
    (void)len;
    if (kind == kAttnQ8Mfma) return 64;
    return kind == kAttnBF16Mfma ? 64 : 128;
}
long plan_rows(int kind, const int *lens, int n, int ncu) {
    const long chunk = plan_chunk(kind);
    const long target = n == 1 ? lone_splits(kind, lens[0]) : (long)plan_wg_per_cu(kind) * ncu;
    auto count = [&](long r) {
        long c = 0;
        for (int i = 0; i < n; ++i) c += nsplit_of(kind, lens[i], r);
        return c;
    };
    long lo = n == 1 ? 2 : 4, hi = lo;  // in chunks
    for (int i = 0; i < n; ++i) hi = std::max(hi, ((long)lens[i] + chunk - 1) / chunk);
    while (lo < hi) {  // count() does not increase with r
        const long mid = (lo + hi) / 2;
        if (count(mid * chunk) <= target) hi = mid;
        else lo = mid + 1;
    }
    long r = lo * chunk;
    if (kind == kAttnQ8Mfma) r = std::min<long>(r, 1024L);
    return r;
}

// Rows per split of one sequence under the launch's r. Q8: r (the last split takes the rest).
// Other kinds: the sequence's nsplit_of(len, r) splits made equal (ceil(len / n) rows, rounded
// up to the chunk), so its longest split is not longer than r. At most kMaxSplits splits per
// sequence (the combine's per-split staging): very long histories get longer splits.
long seq_rows(int kind, long len, long r) {
    const long chunk = plan_chunk(kind), rmin = (len + kMaxSplits - 1) / kMaxSplits;
    long rps = r;
    if (kind != kAttnQ8Mfma) {
        const long n = nsplit_of(kind, len, r);
        rps = ((len + n - 1) / n + chunk - 1) / chunk * chunk;
    }
    return rps < rmin ? (rmin + chunk - 1) / chunk * chunk : rps;
}

// Attention plan of a launch group: the per-sequence descriptors with their split-K layout,
// and the device scratch it needs. solo: every sequence gets the plan it would get alone in
// the launch, so its result does not depend on the other members (block decode).
struct GroupPlan {
    SeqTable t;
    int kind = 0, rps = 0, total_splits = 0, lmax = 0;
    size_t part_bytes = 0, scores_bytes = 0;
};

void plan_group(int fmt, const Dims &d, const SeqIn *seqs, int B, bool solo, GroupPlan &p) {
    const int ncu = ctx().ncu;
    const bool kimi = kimi_attn(d) && fmt != kFmtExp;
    p.kind = !kimi ? kAttnGeneric : fmt == kFmtQ8 ? kAttnQ8Mfma : fmt == kFmtBF16 ? kAttnBF16Mfma : kAttnF32Mfma;
    SeqTable &t = p.t;
    memset(&t, 0, sizeof t);
    t.n = B;
    p.lmax = 0;
    for (int i = 0; i < B; ++i) {
        SeqDesc &s = t.s[i];
        s.a = seqs[i].m->a;
        s.b = seqs[i].m->b;
        s.c = seqs[i].m->c;
        s.pos = seqs[i].pos;
        s.len = seqs[i].pos + 1;
        p.lmax = std::max(p.lmax, s.len);
    }
    p.rps = 0;
    p.total_splits = 0;
    if (p.kind == kAttnGeneric) {
        for (int i = 0; i < B; ++i) {
            t.s[i].split0 = fmt == kFmtExp ? i * d.NH : i;
            t.s[i].nsplit = 1;
        }
        p.total_splits = fmt == kFmtExp ? B * d.NH : B;
    } else {
        int lens[kMaxBatch];
        for (int i = 0; i < B; ++i) lens[i] = t.s[i].len;
        const long r = solo ? 0 : plan_rows(p.kind, lens, B, ncu);
        for (int i = 0; i < B; ++i) {
            SeqDesc &s = t.s[i];
            s.split0 = p.total_splits;
            s.rps = (int)seq_rows(p.kind, s.len, solo ? plan_rows(p.kind, &lens[i], 1, ncu) : r);
            s.nsplit = (int)nsplit_of(p.kind, s.len, s.rps);
            p.total_splits += s.nsplit;
            p.rps = std::max(p.rps, s.rps);
        }
    }
    const int G = fmt == kFmtExp ? 1 : d.NH;
    const int DVm = fmt == kFmtExp ? d.DV : d.R;
    p.part_bytes = (size_t)p.total_splits * G * (DVm + 2) * sizeof(float);
    const int P = fmt == kFmtExp ? B * d.NH : B;
    p.scores_bytes = p.kind == kAttnGeneric ? (size_t)P * G * p.lmax * sizeof(float) : 0;
}

// Everything the launch groups of a call need, acquired before any group launches, so that a
// failure (an allocation) leaves every state unchanged: the device copies of all states, the
// workspace of the largest group, the partials and score scratch of the most demanding group,
// and the RoPE table up to the largest position.
template <class S>
int prepare_groups(int fmt, const Dims &d, float theta, S *const *states, int B, size_t rb,
                   std::vector<Mirror *> &ms) {
    Ctx &c = ctx();
    ms.assign(B, nullptr);
    int maxpos = 0;
    for (int i = 0; i < B; ++i) {
        if (mirror_get(states[i], view_of(states[i]), &ms[i]) != 0) return -1;
        maxpos = std::max(maxpos, states[i]->len);
    }
    const float2 *cs = nullptr;
    if (rope_table(theta, d.DR, maxpos + 1, &cs) != 0) return -1;
    DecodeWork wk;
    if (decode_work(d, std::min(B, kMaxBatch), (int)rb, wk) != 0) return -1;
    size_t part = 0, scores = 0;
    for (int g0 = 0; g0 < B; g0 += kMaxBatch) {
        const int n = std::min(kMaxBatch, B - g0);
        SeqIn seqs[kMaxBatch];
        for (int i = 0; i < n; ++i) seqs[i] = {ms[g0 + i], states[g0 + i]->len};
        GroupPlan gp;
        plan_group(fmt, d, seqs, n, false, gp);
        part = std::max(part, gp.part_bytes);
        scores = std::max(scores, gp.scores_bytes);
    }
    float *pp = nullptr;
    if (reserve_part(part, &pp) != 0) return -1;
    if (c.scores.bytes < scores) {
        if (c.capturing) {
            set_err("score scratch growth during graph capture");
            return -1;
        }
        if (dev_reserve(c.scores, scores) != 0) return -1;
    }
    return 0;
}

// One decode step for a group of B <= kMaxBatch sequences whose mirrors are synced.
// d_x: device input rows [B,H]; d_out: device output rows [B,H]. Rows appended on the device
// at each pos; staged copies in w.rows. solo: see plan_group.
// part_cap > 0: w.part is a caller-provided buffer of part_cap bytes for the split partials and
// nothing is allocated (the RoPE table must already cover the positions).
int decode_group(int fmt, const Dims &d, float eps, float theta, const DevWeights &dw,
                 const SeqIn *seqs, int B, const float *d_x, float *d_out, bool residual,
                 DecodeWork &w, bool solo = false, size_t part_cap = 0) {
    Ctx &c = ctx();
    hipStream_t st = c.stream;
    int maxpos = 0;
    for (int i = 0; i < B; ++i) maxpos = std::max(maxpos, seqs[i].pos);
    const float2 *cs = nullptr;
    if ((part_cap ? rope_lookup(theta, d.DR, maxpos + 1, &cs) : rope_table(theta, d.DR, maxpos + 1, &cs)) != 0)
        return -1;

    GroupPlan gp;
    plan_group(fmt, d, seqs, B, solo, gp);
    SeqTable &t = gp.t;
    const int kind = gp.kind, rps = gp.rps, total_splits = gp.total_splits, lmax = gp.lmax;
    const size_t part_bytes = gp.part_bytes;
    if (part_cap) {
        if (part_bytes > part_cap || kind == kAttnGeneric) {
            set_err("the split plan needs %zu bytes of partials; the fixed scratch holds %zu (%d splits)",
                    part_bytes, part_cap, total_splits);
            return -1;
        }
    } else if (reserve_part(part_bytes, &w.part) != 0) {
        return -1;
    }
    if (kind == kAttnGeneric) {
        const size_t bytes = gp.scores_bytes;
        if (c.scores.bytes < bytes) {
            if (c.capturing) {
                set_err("score scratch growth during graph capture");
                return -1;
            }
            if (dev_reserve(c.scores, bytes) != 0) return -1;
        }
        w.scores = (float *)c.scores.p;
    }

    const int ldy = d.QO + d.KVO;
    // The fused form (see FqArgs): Q8 MFMA attention of independent sequences (no block members)
    // at the Kimi shapes, one round of workgroups with room for the 17 B producer tasks, the
    // k-split projection, W_UK^T in fragment order; the no-allocation entry point keeps the
    // two-launch form. Measured with the query preparation alone inside (headline stack, 8 x 32K
    // Q8 rows, 27 layers): 1.522 -> 1.483 ms per step.
    const bool fuse_base = c.fq_on && fmt == kFmtQ8 && kind == kAttnQ8Mfma && !solo && part_cap == 0 &&
                           kimi_attn(d) && d.DN == 128 && d.QD == 192 && gemv_ksplit_ok(d.H, d.H) && ukt_shape(d) &&
                           dw.ukt && 17 * B <= total_splits && total_splits <= c.ncu && c.fq_flags && c.fq_err;
    // ... and the q_proj | kv_a projection inside it too (fq_gemv): at most eight sequences, x
    // 16-byte aligned, a launch of max(splits, kGemvTasks) <= CU count workgroups.
    const bool pfuse_ok = fuse_base && c.gemv_on && gemv_fuse_ok(d, B) && gemv_ksplit_ok(d.H, d.H) &&
                          ((uintptr_t)d_x % 16) == 0 && std::max(total_splits, kGemvTasks) <= c.ncu;
    // ... and the combine inside it (q8_comb_tail): eight sequences (or a multiple) with equal
    // split counts, each sequence's splits on one XCD (kCombXcd); or sequences of 16 or more
    // splits each, their partials exchanged past the L2s (kCombCross). Measured (headline
    // stack, lone decodes): see the design notes on the fused combine.
    const bool comb_shape = c.comb_on && combine_writes_hos(fmt, d) && gemv_xs_ok(d.HO);
    const int comb_mode = !comb_shape ? 0 : comb_ok(t, d, total_splits) ? 1 : comb_cross_ok(t, d) ? 2 : 0;
    // A lone sequence takes the fused form only with the projection and the combine inside it
    // (with the query preparation alone its 17 producer tasks held up its 64 short splits: a
    // lone 8K-row decode 29.5 -> 30.5 us).
    const bool fuse = fuse_base && (B >= 2 || (pfuse_ok && comb_mode != 0));
    const bool pfuse = fuse && pfuse_ok;
    const int comb = fuse ? comb_mode : 0;
    {
        // q_proj | kv_a: k split over kGemvKs blocks where the shape allows (the consumers
        // add the partials), else one pass
        StageTimer tm(pfuse ? -1 : 0);
        if (pfuse) {
            w.ynp = kGemvKs;
            w.ypstride = (size_t)B * ldy;
        } else if (gemv_ksplit_ok(d.H, d.H)) {
            if (((uintptr_t)d_x % 16) != 0) {  // the kernel reads 16-byte vectors
                HIP_TRY(hipMemcpyAsync(w.x, d_x, (size_t)B * d.H * sizeof(float), hipMemcpyDeviceToDevice, st));
                d_x = w.x;
            }
            w.ynp = kGemvKs;
            w.ypstride = (size_t)B * ldy;
            HIP_TRY(launch_gemv_ksplit(st, w.y, w.ypstride, ldy, d_x, d.H, B, dw.q, d.QO, dw.kva,
                                       d.KVO, d.H, fuse ? c.fq_flags : nullptr, fuse ? kFqFlagLines : 0));
        } else {
            w.ynp = 1;
            w.ypstride = 0;
            HIP_TRY(launch_gemv(st, w.y, ldy, d_x, d.H, B, dw.q, d.QO, dw.kva, d.KVO, d.H, false));
        }
    }
    if (fmt == kFmtExp) {
        {
            StageTimer tm(1);
            HIP_TRY(launch_append(st, fmt, t, d, w.y, ldy, d.QO, w.ynp, w.ypstride, dw.norm, eps, cs,
                                  w, false, 0));
            HIP_TRY(launch_gemv(st, w.kv, d.KVB, w.latent, d.R, B, dw.kvb, d.KVB, nullptr, 0, d.R, false));
            HIP_TRY(launch_store_expanded(st, t, d, w));
        }
        {
            StageTimer tm(2);
            HIP_TRY(launch_qprep(st, fmt, t, d, dw.kvb, cs, w, false));
        }
    } else if (!fuse) {
        // append and query preparation in one launch (timed as stage 1)
        StageTimer tm(1);
        HIP_TRY(launch_append_qprep(st, fmt, t, d, w.y, ldy, d.QO, w.ynp, w.ypstride, dw.norm, eps, cs, dw.kvb,
                                    dw.ukt, w, kind == kAttnQ8Mfma));
    }
    if (pfuse && c.fq_dirty) {
        HIP_TRY(launch_clear_flags(st, c.fq_flags, kFqFlagLines));
        c.fq_dirty = false;
    }
    {
        StageTimer tm(3);
        FqArgs fq{};
        if (fuse) {
            fq.y = w.y;
            fq.ukt = dw.ukt;
            fq.cs = cs;
            fq.norm = dw.norm;
            fq.rows = w.rows;
            fq.flags = c.fq_flags;
            fq.err = c.fq_err;
            fq.pstride = w.ypstride;
            fq.ldy = ldy;
            fq.koff = d.QO;
            fq.row_bytes = d.R + 4 + 2 * d.DR;
            fq.eps = eps;
            fq.splits = total_splits;
            fq.spin = c.fq_spin;
            if (comb) {
                fq.comb = comb;
                fq.kvb = dw.kvb;
                fq.ho = w.ho;
                fq.hos = w.hos;
            }
            if (pfuse) {
                fq.gemv = 1;
                fq.x = d_x;
                fq.wq = dw.q;
                fq.wkva = dw.kva;
                fq.ldx = d.H;
                fq.in = d.H;
                fq.out0 = d.QO;
                fq.out1 = d.KVO;
            }
        }
        if (fuse) c.fq_dirty = true;
        HIP_TRY(launch_attention(st, kind, fmt, t, d, rps, total_splits, lmax, w, solo ? B : 0, fuse ? &fq : nullptr));
    }
    if (!comb) {
        StageTimer tm(4);
        HIP_TRY(launch_combine(st, fmt, t, d, dw.kvb, w));
    }
    {
        // o_proj: from the bf16 hi | lo planes of the head outputs when combine wrote them
        StageTimer tm(5);
        // after a fused launch, o_proj clears its flags for the next one (a fused launch that
        // computes the projection itself has no q_proj | kv_a launch before it to do so)
        if (combine_writes_hos(fmt, d) && gemv_xs_ok(d.HO)) {
            HIP_TRY(launch_gemv_xs(st, d_out, d.H, w.hos, B, dw.o, d.H, d.HO, residual, fuse ? c.fq_flags : nullptr,
                                   fuse ? kFqFlagLines : 0));
            if (fuse) c.fq_dirty = false;
        } else {
            HIP_TRY(launch_gemv(st, d_out, d.H, w.ho, d.HO, B, dw.o, d.H, nullptr, 0, d.HO, residual));
        }
    }
    return 0;
}

// Write staged appended rows (device w.rows) back into the host arrays.
void write_back_rows(int fmt, const HostView &v, int pos, const uint8_t *row) {
    if (fmt == kFmtQ8) {
        const int R = v.d0, DR = v.d1;
        memcpy((int8_t *)v.ha + (size_t)pos * R, row, (size_t)R);
        memcpy((float *)v.hb + pos, row + R, 4);
        memcpy((uint16_t *)v.hc + (size_t)pos * DR, row + R + 4, 2 * (size_t)DR);
    } else if (fmt == kFmtF32) {
        const int R = v.d0, DR = v.d1;
        memcpy((float *)v.ha + (size_t)pos * R, row, 4 * (size_t)R);
        memcpy((float *)v.hb + (size_t)pos * DR, row + 4 * (size_t)R, 4 * (size_t)DR);
    } else if (fmt == kFmtBF16) {
        const int R = v.d0, DR = v.d1;
        memcpy((uint16_t *)v.ha + (size_t)pos * R, row, 2 * (size_t)R);
        memcpy((uint16_t *)v.hb + (size_t)pos * DR, row + 2 * (size_t)R, 2 * (size_t)DR);
    } else {
        const size_t nk = (size_t)v.d0 * v.d1, nv = (size_t)v.d0 * v.d2;
        memcpy((float *)v.ha + (size_t)pos * nk, row, 4 * nk);
        memcpy((float *)v.hb + (size_t)pos * nv, row + 4 * nk, 4 * nv);
    }
}

// Validation shared by the host-API decode entry points (reference conditions:
// src/mla_compressed_q8_state.c:167-180).
template <class S>
bool state_dims_ok(const S *s, const KvlMlaConfig *cfg);
template <>
bool state_dims_ok(const KvlMlaCompressedQ8State *s, const KvlMlaConfig *cfg) {
    return s->kv_lora_rank == cfg->kv_lora_rank && s->qk_rope_dim == cfg->qk_rope_dim;
}
template <>
bool state_dims_ok(const KvlMlaCompressedState *s, const KvlMlaConfig *cfg) {
    return s->kv_lora_rank == cfg->kv_lora_rank && s->qk_rope_dim == cfg->qk_rope_dim;
}
template <>
bool state_dims_ok(const KvlMlaCompressedBF16State *s, const KvlMlaConfig *cfg) {
    return s->kv_lora_rank == cfg->kv_lora_rank && s->qk_rope_dim == cfg->qk_rope_dim;
}
template <>
bool state_dims_ok(const KvlMlaState *s, const KvlMlaConfig *cfg) {
    return s->num_heads == cfg->num_heads && s->qk_nope_dim == cfg->qk_nope_dim &&
           s->qk_rope_dim == cfg->qk_rope_dim && s->v_head_dim == cfg->v_head_dim;
}

template <class S>
int fmt_of();
template <>
int fmt_of<KvlMlaCompressedQ8State>() { return kFmtQ8; }
template <>
int fmt_of<KvlMlaCompressedState>() { return kFmtF32; }
template <>
int fmt_of<KvlMlaCompressedBF16State>() { return kFmtBF16; }
template <>
int fmt_of<KvlMlaState>() { return kFmtExp; }

// Host-buffer decode of one token for each of B sequences (any B). positions[i] == len.
template <class S>
int decode_host(float *out, const float *x, const int *positions, int B, const KvlMlaConfig *cfg,
                const KvlMlaBF16 *w, S *const *states) {
    Dims d;
    if (!out || !x || B <= 0 || !states || !weights_ok(w) || !dims_of(cfg, d)) {
        set_err("invalid arguments");
        return -1;
    }
    for (int i = 0; i < B; ++i) {
        const S *s = states[i];
        const int pos = positions ? positions[i] : (s ? s->len : -1);
        if (!s || pos != s->len || pos < 0 || pos >= s->capacity || !state_dims_ok(s, cfg)) {
            set_err("sequence %d: position/capacity/dims check failed", i);
            return -1;
        }
    }
    if (!dims_supported(d)) return -1;
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    const int fmt = fmt_of<S>();
    DevWeights dw;
    if (dev_weights(w, d, dw) != 0) return -1;
    const size_t rb = fmt == kFmtExp ? row_bytes_of(fmt, d.NH, d.QD, d.DV)
                                     : row_bytes_of(fmt, d.R, d.DR, 0);
    std::vector<Mirror *> ms;
    if (prepare_groups(fmt, d, cfg->rope_theta, states, B, rb, ms) != 0) return -1;
    if (pin_reserve(c.pin_in, (size_t)std::min(B, kMaxBatch) * d.H * sizeof(float)) != 0 ||
        pin_reserve(c.pin_out, (size_t)std::min(B, kMaxBatch) * (d.H * sizeof(float) + rb)) != 0)
        return -1;
    for (int g0 = 0; g0 < B; g0 += kMaxBatch) {
        const int n = std::min(kMaxBatch, B - g0);
        DecodeWork wk;
        if (decode_work(d, n, (int)rb, wk) != 0) return -1;
        SeqIn seqs[kMaxBatch];
        for (int i = 0; i < n; ++i) seqs[i] = {ms[g0 + i], states[g0 + i]->len};
        const size_t xin = (size_t)n * d.H * sizeof(float);
        const size_t outb = xin + (size_t)n * rb;
        if (pin_reserve(c.pin_in, xin) != 0 || pin_reserve(c.pin_out, outb) != 0) return -1;
        memcpy(c.pin_in.p, x + (size_t)g0 * d.H, xin);
        // The kernels read x from and write the output (and, for the compressed formats, the
        // appended rows) to the pinned host buffers directly: three copy launches fewer per call.
        // The expanded format's store kernel reads its staged rows back, so they stay on the device.
        float *pout = (float *)c.pin_out.p;
        uint8_t *prows = (uint8_t *)c.pin_out.p + xin;
        if (fmt != kFmtExp) wk.rows = prows;
        if (decode_group(fmt, d, cfg->rms_eps, cfg->rope_theta, dw, seqs, n, (const float *)c.pin_in.p, pout,
                         false, wk) != 0)
            return -1;
        if (fmt == kFmtExp)
            HIP_TRY(hipMemcpyAsync(prows, wk.rows, (size_t)n * rb, hipMemcpyDeviceToHost, c.stream));
        HIP_TRY(hipStreamSynchronize(c.stream));
        if (*c.fq_err) {
            *c.fq_err = 0;
            c.fq_dirty = true;  // a timed-out wait may have left its counters behind
            set_err("a wait of the fused query preparation timed out (results invalid); "
                    "KVL_MLA_NO_FUSED_QPREP=1 selects the two-launch form");
            return -1;
        }
        memcpy(out + (size_t)g0 * d.H, c.pin_out.p, xin);
        for (int i = 0; i < n; ++i) {
            S *s = states[g0 + i];
            const int pos = s->len;
            write_back_rows(fmt, view_of(s), pos, (const uint8_t *)c.pin_out.p + xin + (size_t)i * rb);
            s->len = pos + 1;
            seqs[i].m->synced = s->len;
        }
    }
    return 0;
}

template <class S>
int decode_device(float *d_out, const float *d_x, int B, const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                  S *const *states, unsigned flags);

// The attention half of a decoder layer (src/generate.c:34-67, attention_token) for a batch,
// stream-ordered over device buffers: n1 = RMSNorm(h, input_norm) (src/ops.c:76-83 rounding),
// h += attention(n1) with each sequence's row appended, n2 = RMSNorm(h, post_attn_norm) for
// the MLP. The residual add is the o_proj kernel's accumulate: h + o, as the reference's
// r1[i] = x[i] + attn[i].
template <class S>
int attention_layer_device(float *d_h, float *d_n2, int B, const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                           const uint16_t *input_norm, const uint16_t *post_norm, S *const *states,
                           unsigned flags) {
    if (!d_h || !d_n2 || d_n2 == d_h || B <= 0 || !cfg || !input_norm || !post_norm || cfg->hidden_size <= 0) {
        set_err("invalid arguments");
        return -1;
    }
    if (flags & ~(unsigned)KVL_MLA_NO_ADVANCE) {
        set_err("unsupported flags (the residual add is implied)");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    const int H = cfg->hidden_size;
    const uint16_t *din = nullptr, *dpost = nullptr;
    if (dev_weight(input_norm, (size_t)H, &din) != 0 || dev_weight(post_norm, (size_t)H, &dpost) != 0) return -1;
    const size_t need = (size_t)B * H * sizeof(float);
    if (c.layer.bytes < need) {
        if (c.capturing) {
            set_err("layer workspace growth during graph capture");
            return -1;
        }
        if (dev_reserve(c.layer, need) != 0) return -1;
    }
    float *n1 = (float *)c.layer.p;
    HIP_TRY(launch_rmsnorm(c.stream, n1, d_h, din, H, B, cfg->rms_eps));
    if (decode_device(d_h, n1, B, cfg, w, states, flags | KVL_MLA_RESIDUAL) != 0) return -1;
    HIP_TRY(launch_rmsnorm(c.stream, d_n2, d_h, dpost, H, B, cfg->rms_eps));
    return 0;
}

// Block decode of `count` tokens of one sequence (src/mla_compressed_state.c:163-184 loops the
// single-token decode). Here the tokens run through the batched path as members that share the
// state: member t sits at position start + t and gets the split plan a lone decode at that
// position gets. Each stage computes a member exactly as a lone decode computes its token (the
// projections, the append, the attention splits, the combine and o_proj depend only on that
// member's inputs and rows), and a group's rows are all appended before its attention reads
// them (member t reads rows [0, start + t]). Outputs and rows therefore equal the serial
// loop's bit for bit; the launches and the history reads of a group are shared.
template <class S>
int decode_block(float *out, const float *x, int count, int start, const KvlMlaConfig *cfg,
                 const KvlMlaBF16 *w, S *state) {
    Dims d;
    if (!out || !x || !cfg || !w || !state || count <= 0 || start != state->len || start < 0 ||
        count > state->capacity - start) {
        set_err("invalid arguments");
        return -1;
    }
    if (!weights_ok(w) || !dims_of(cfg, d) || !state_dims_ok(state, cfg)) {
        set_err("invalid config, weights or state dims");
        return -1;
    }
    if (!dims_supported(d)) return -1;
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    const int fmt = fmt_of<S>();
    DevWeights dw;
    if (dev_weights(w, d, dw) != 0) return -1;
    const size_t rb = row_bytes_of(fmt, d.R, d.DR, 0);
    Mirror *m = nullptr;
    if (mirror_get(state, view_of(state), &m) != 0) return -1;
    for (int t0 = 0; t0 < count;) {
        // members of this group: at most kMaxBatch
        const int n = std::min(kMaxBatch, count - t0);
        DecodeWork wk;
        if (decode_work(d, n, (int)rb, wk) != 0) return -1;
        SeqIn seqs[kMaxBatch];
        for (int i = 0; i < n; ++i) seqs[i] = {m, start + t0 + i};
        const size_t xin = (size_t)n * d.H * sizeof(float);
        if (pin_reserve(c.pin_in, xin) != 0 || pin_reserve(c.pin_out, xin + (size_t)n * rb) != 0) return -1;
        memcpy(c.pin_in.p, x + (size_t)t0 * d.H, xin);
        // x, the outputs and the appended rows in the pinned host buffers, as in decode_host
        wk.rows = (uint8_t *)c.pin_out.p + xin;
        if (decode_group(fmt, d, cfg->rms_eps, cfg->rope_theta, dw, seqs, n, (const float *)c.pin_in.p,
                         (float *)c.pin_out.p, false, wk, true) != 0)
            return -1;
        HIP_TRY(hipStreamSynchronize(c.stream));
        memcpy(out + (size_t)t0 * d.H, c.pin_out.p, xin);
        const HostView v = view_of(state);
        for (int i = 0; i < n; ++i)
            write_back_rows(fmt, v, start + t0 + i, (const uint8_t *)c.pin_out.p + xin + (size_t)i * rb);
        state->len = start + t0 + n;
        m->synced = state->len;
        t0 += n;
    }
    return 0;
}

// Stream-ordered decode over device buffers (bound weights, synced mirrors).
template <class S>
int decode_device(float *d_out, const float *d_x, int B, const KvlMlaConfig *cfg,
                  const KvlMlaBF16 *w, S *const *states, unsigned flags) {
    Dims d;
    if (!d_out || !d_x || B <= 0 || !states || !weights_ok(w) || !dims_of(cfg, d)) {
        set_err("invalid arguments");
        return -1;
    }
    for (int i = 0; i < B; ++i) {
        const S *s = states[i];
        if (!s || s->len < 0 || s->len >= s->capacity || !state_dims_ok(s, cfg)) {
            set_err("sequence %d: capacity/dims check failed", i);
            return -1;
        }
    }
    if (!dims_supported(d)) return -1;
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    const int fmt = fmt_of<S>();
    DevWeights dw;
    if (dev_weights(w, d, dw) != 0) return -1;
    const size_t rb = row_bytes_of(fmt, d.R, d.DR, 0);
    std::vector<Mirror *> ms;
    if (prepare_groups(fmt, d, cfg->rope_theta, states, B, rb, ms) != 0) return -1;
    for (int g0 = 0; g0 < B; g0 += kMaxBatch) {
        const int n = std::min(kMaxBatch, B - g0);
        DecodeWork wk;
        if (decode_work(d, n, (int)rb, wk) != 0) return -1;
        SeqIn seqs[kMaxBatch];
        for (int i = 0; i < n; ++i) seqs[i] = {ms[g0 + i], states[g0 + i]->len};
        if (decode_group(fmt, d, cfg->rms_eps, cfg->rope_theta, dw, seqs, n, d_x + (size_t)g0 * d.H,
                         d_out + (size_t)g0 * d.H, (flags & KVL_MLA_RESIDUAL) != 0, wk) != 0)
            return -1;
        if (!(flags & KVL_MLA_NO_ADVANCE)) {
            for (int i = 0; i < n; ++i) {
                S *s = states[g0 + i];
                s->len += 1;
                seqs[i].m->synced = s->len;  // host rows of the new position are not written
            }
        }
    }
    (void)c;
    return 0;
}

// Decode of decode_device's arithmetic (Q8 histories, the MFMA route) that allocates nothing:
// the workspace and the partials live in the device array `scratch`; the weights must be bound,
// every state's device copy must exist and hold its rows [0, len), and the RoPE table must
// cover the positions. Rows appended at len stay on the device; len advances unless
// KVL_MLA_NO_ADVANCE. Two calls on one GPU share the array, so calls that overlap in time on
// that GPU (graph launches on other streams) race.
int decode_q8_noalloc(float *d_out, const float *d_x, int B, const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                      KvlMlaCompressedQ8State *const *states, unsigned flags) {
    Dims d;
    if (!d_out || !d_x || B <= 0 || !states || !weights_ok(w) || !dims_of(cfg, d)) {
        set_err("invalid arguments");
        return -1;
    }
    if (B > kNoAllocMaxBatch) {
        set_err("batch %d exceeds the %d sequences of the fixed scratch", B, kNoAllocMaxBatch);
        return -1;
    }
    if (flags & ~(unsigned)(KVL_MLA_RESIDUAL | KVL_MLA_NO_ADVANCE)) {
        set_err("unsupported flags");
        return -1;
    }
    if (!kimi_attn(d) || !dims_supported(d)) {
        set_err("dims outside the MFMA route (16 heads, kv_lora_rank 512, qk_rope_dim 64)");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != c.device || !g_scratch[dev]) {
        set_err("current device %d is not the library's device %d", dev, c.device);
        return -1;
    }
    DevWeights dw;
    const uint16_t **slot[5] = {&dw.q, &dw.kva, &dw.norm, &dw.kvb, &dw.o};
    const uint16_t *host[5] = {w->q_proj, w->kv_a_proj, w->kv_a_norm, w->kv_b_proj, w->o_proj};
    const size_t elems[5] = {(size_t)d.QO * d.H, (size_t)d.KVO * d.H, (size_t)d.R, (size_t)d.KVB * d.R,
                             (size_t)d.H * d.HO};
    for (int k = 0; k < 5; ++k) {
        auto it = c.weights.find(host[k]);
        if (it == c.weights.end() || it->second.pins <= 0 || it->second.bytes != elems[k] * sizeof(uint16_t)) {
            set_err("weights must be bound (kvl_mla_bind_weights) before a no-allocation call");
            return -1;
        }
        *slot[k] = (const uint16_t *)it->second.dev;
        if (k == 3 && ukt_shape(d)) {
            if (!it->second.t_ok) {
                set_err("weights must be bound (kvl_mla_bind_weights) before a no-allocation call");
                return -1;
            }
            dw.ukt = (const uint16_t *)it->second.devt;
        }
    }
    SeqIn seqs[kNoAllocMaxBatch];
    for (int i = 0; i < B; ++i) {
        KvlMlaCompressedQ8State *s = states[i];
        if (!s || s->len < 0 || s->len >= s->capacity || !state_dims_ok(s, cfg)) {
            set_err("sequence %d: capacity/dims check failed", i);
            return -1;
        }
        const HostView v = view_of(s);
        auto it = c.mirrors.find(s);
        if (it == c.mirrors.end() || it->second.fmt != v.fmt || it->second.ha != v.ha || it->second.hb != v.hb ||
            it->second.hc != v.hc || it->second.capacity != v.capacity || it->second.d0 != v.d0 ||
            it->second.d1 != v.d1 || it->second.synced < s->len) {
            set_err("sequence %d: the state's rows [0, len) are not on the device (an allocating call or "
                    "*_fill_synthetic puts them there)", i);
            return -1;
        }
        seqs[i] = {&it->second, s->len};
    }
    DecodeWork wk;
    const size_t rb = row_bytes_of(kFmtQ8, d.R, d.DR, 0);
    const size_t wbytes = decode_work_at(d, B, (int)rb, nullptr, wk);
    if (wbytes >= kNoAllocScratchBytes) {
        set_err("the decode workspace (%zu bytes) exceeds the fixed scratch (%zu bytes)", wbytes,
                kNoAllocScratchBytes);
        return -1;
    }
    char *base = (char *)g_scratch[dev];
    decode_work_at(d, B, (int)rb, base, wk);
    wk.part = (float *)(base + wbytes);
    if (decode_group(kFmtQ8, d, cfg->rms_eps, cfg->rope_theta, dw, seqs, B, d_x, d_out,
                     (flags & KVL_MLA_RESIDUAL) != 0, wk, false, kNoAllocScratchBytes - wbytes) != 0)
        return -1;
    if (!(flags & KVL_MLA_NO_ADVANCE)) {
        for (int i = 0; i < B; ++i) {
            states[i]->len += 1;
            seqs[i].m->synced = states[i]->len;
        }
    }
    return 0;
}

// What a state fill needs on the device: dims, the kv_a weight and norm, the RoPE table, the
// state's device mirror.
struct FillCtx {
    Dims d{};
    int fmt = 0;
    float eps = 0.f;
    const uint16_t *kva = nullptr, *norm = nullptr;
    const float2 *cs = nullptr;
    Mirror *m = nullptr;
};

// Checks of src/mla_compressed_state.c:52-66 / src/mla_compressed_q8_state.c:129-140 (empty
// state, seq_len within capacity, matching dims) and the device set-up of a fill.
template <class S>
int fill_begin(int seq_len, const KvlMlaConfig *cfg, const KvlMlaBF16 *w, S *s, FillCtx &f) {
    if (!cfg || !w || !s || !w->kv_a_proj || !w->kv_a_norm || seq_len <= 0 || s->len != 0 ||
        seq_len > s->capacity || !state_dims_ok(s, cfg)) {
        set_err("invalid arguments");
        return -1;
    }
    const int H = cfg->hidden_size, R = cfg->kv_lora_rank, DR = cfg->qk_rope_dim;
    if (H <= 0 || R <= 0 || DR <= 0 || (DR & 1) || !(cfg->rope_theta > 0.0f)) {
        set_err("invalid config");
        return -1;
    }
    if (R > 1024 || DR > 256) {
        set_err("dims beyond the device kernels' bounds");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    f.fmt = fmt_of<S>();
    f.eps = cfg->rms_eps;
    f.d.H = H;
    f.d.R = R;
    f.d.DR = DR;
    f.d.KVO = R + DR;
    f.d.NH = 1;
    if (dev_weight(w->kv_a_proj, (size_t)f.d.KVO * H, &f.kva) != 0) return -1;
    if (dev_weight(w->kv_a_norm, (size_t)R, &f.norm) != 0) return -1;
    if (mirror_get(s, view_of(s), &f.m) != 0) return -1;
    if (rope_table(cfg->rope_theta, DR, seq_len, &f.cs) != 0) return -1;
    return 0;
}

// Rows [t0, t0 + n) of the state from the kv_a projection of those tokens on the device (np
// partials pstride floats apart, token i at y + i * ldy): the append kernel in rows mode
// (RMSNorm, RoPE, the state's row format) writes the device mirror and stages the rows in
// c.fill; with host_rows they are also copied into the host arrays (synchronous).
template <class S>
int fill_rows(S *s, const FillCtx &f, const float *y, int ldy, int np, size_t pstride, int t0, int n,
              bool host_rows) {
    Ctx &c = ctx();
    const size_t rb = row_bytes_of(f.fmt, f.d.R, f.d.DR, 0);
    if (dev_reserve(c.fill, (size_t)n * rb) != 0) return -1;
    uint8_t *drows = (uint8_t *)c.fill.p;
    SeqTable t;
    memset(&t, 0, sizeof t);
    t.n = 1;
    t.s[0].a = f.m->a;
    t.s[0].b = f.m->b;
    t.s[0].c = f.m->c;
    t.s[0].pos = t0;
    DecodeWork wk{};
    wk.rows = drows;
    HIP_TRY(launch_append(c.stream, f.fmt, t, f.d, y, ldy, 0, np, pstride, f.norm, f.eps, f.cs, wk, false, n));
    if (!host_rows) return 0;
    if (pin_reserve(c.pin_out, (size_t)n * rb) != 0) return -1;
    HIP_TRY(hipMemcpyAsync(c.pin_out.p, drows, (size_t)n * rb, hipMemcpyDeviceToHost, c.stream));
    HIP_TRY(hipStreamSynchronize(c.stream));
    const HostView v = view_of(s);
    for (int i = 0; i < n; ++i) write_back_rows(f.fmt, v, t0 + i, (const uint8_t *)c.pin_out.p + (size_t)i * rb);
    return 0;
}

// kv_a of n tokens from device x [n, H] with the decode path's arithmetic -- the k-split
// partials (launch_kva_tok over the bf16 planes of x) where the decode uses them, else the
// plain GEMV -- so the rows equal those a decode of the same tokens appends; then fill_rows.
// ws: fill_x_bytes(d, n) bytes of device memory, 256-byte aligned.
size_t fill_x_bytes(const Dims &d, int n) {
    const bool ks = gemv_ksplit_ok(d.H, d.H);
    Layout L;
    L.take<uint16_t>(nullptr, ks ? 2 * (size_t)n * d.H : 0);
    L.take<float>(nullptr, (size_t)(ks ? kGemvKs : 1) * n * d.KVO);
    return L.off;
}

template <class S>
int fill_from_x(S *s, const FillCtx &f, const float *dx, void *ws, int t0, int n, bool host_rows) {
    Ctx &c = ctx();
    const Dims &d = f.d;
    const bool ks = gemv_ksplit_ok(d.H, d.H);
    const int np = ks ? kGemvKs : 1;
    Layout L;
    uint16_t *xs = L.take<uint16_t>((char *)ws, ks ? 2 * (size_t)n * d.H : 0);
    float *dy = L.take<float>((char *)ws, (size_t)np * n * d.KVO);
    if (ks) {
        uint16_t *xl = xs + (size_t)n * d.H;
        HIP_TRY(launch_split(c.stream, dx, d.H, xs, xl, d.H, n, d.H));
        HIP_TRY(launch_kva_tok(c.stream, dy, (size_t)n * d.KVO, d.KVO, xs, xl, n, f.kva, d.KVO, d.H));
    } else {
        for (int b0 = 0; b0 < n; b0 += 16 * 65535) {
            const int nb = std::min(n - b0, 16 * 65535);
            HIP_TRY(launch_gemv(c.stream, dy + (size_t)b0 * d.KVO, d.KVO, dx + (size_t)b0 * d.H, d.H, nb, f.kva,
                                d.KVO, nullptr, 0, d.H, false));
        }
    }
    return fill_rows(s, f, dy, d.KVO, np, (size_t)n * d.KVO, t0, n, host_rows);
}

// State prefill-fill (src/mla_compressed_state.c:52-84, src/mla_compressed_q8_state.c:
// 129-159): kv_a of every token, then the append kernel in rows mode, in chunks of 4096 tokens.
template <class S>
int state_prefill(const float *x, int seq_len, const KvlMlaConfig *cfg, const KvlMlaBF16 *w, S *s) {
    FillCtx f;
    if (!x) {
        set_err("invalid arguments");
        return -1;
    }
    if (fill_begin(seq_len, cfg, w, s, f) != 0) return -1;
    Ctx &c = ctx();
    const int H = f.d.H, chunk = 4096;
    for (int t0 = 0; t0 < seq_len; t0 += chunk) {
        const int n = std::min(chunk, seq_len - t0);
        const size_t xb = ((size_t)n * H * sizeof(float) + 255) & ~(size_t)255;
        if (dev_reserve(c.prefill, xb + fill_x_bytes(f.d, n)) != 0) return -1;
        float *dx = (float *)c.prefill.p;
        HIP_TRY(hipMemcpyAsync(dx, x + (size_t)t0 * H, (size_t)n * H * sizeof(float), hipMemcpyHostToDevice,
                               c.stream));
        if (fill_from_x(s, f, dx, (char *)c.prefill.p + xb, t0, n, true) != 0) return -1;
    }
    s->len = seq_len;
    f.m->synced = seq_len;
    return 0;
}

// Causal prefill (src/mla_prefill_streaming.c:78-206). d_x/d_out device buffers.
// host_call: the caller checks the call's range flag itself (host-buffer entry points), else
// the library's sticky flag is raised too. generic: the generic route whatever the dims.
int prefill_device(float *d_out, const float *d_x, int S, const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                   PrefillKva *kva = nullptr, bool host_call = false, bool generic = false) {
    Dims d;
    if (!d_out || !d_x || S <= 0 || !weights_ok(w) || !dims_of(cfg, d)) {
        set_err("invalid arguments");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    DevWeights dw;
    if (dev_weights(w, d, dw) != 0) return -1;
    const float2 *cs = nullptr;
    if (rope_table(cfg->rope_theta, d.DR, S, &cs) != 0) return -1;
    const size_t bytes = prefill_bytes(d, S, generic);
    if (c.scores.bytes < bytes) {
        if (c.capturing) {
            set_err("prefill workspace growth during graph capture");
            return -1;
        }
        if (dev_reserve(c.scores, bytes) != 0) return -1;
    }
    const _Float16 *wo16 = nullptr;
    PrefillRange range;
    range.generic = generic;
    if (prefill_mfma_shape(d) && !generic) {
        int shift = 0;
        if (dev_weight_f16(w->o_proj, (size_t)d.H * d.HO, &wo16, &shift) != 0) return -1;
        range.oscale = ldexpf(1.0f, shift);
        range.vscale = prefill_vscale(w, d);
        if (!host_call) {
            if (!c.rflag.p) {
                if (c.capturing) {
                    set_err("prefill flag allocation during graph capture (run one prefill first)");
                    return -1;
                }
                if (dev_reserve(c.rflag, 256) != 0) return -1;
                HIP_TRY(hipMemsetAsync(c.rflag.p, 0, 256, c.stream));
            }
            range.sticky = (int *)c.rflag.p;
        }
    }
    HIP_TRY(launch_prefill_all(c.stream, d, S, cfg->rms_eps, d_x, d_out, dw.q, dw.kva, dw.norm, dw.kvb,
                               dw.o, wo16, cs, c.scores.p, kva, &range));
    return 0;
}

// After a host-buffer prefill has run on the MFMA route (stream synchronised): when a query row
// fell outside that route's range (the call's flag), the attention output is computed again on
// the generic route (fp32 operands, double score dots) into d_out. The state rows of a prefill
// with state fill do not depend on the attention and stay.
int prefill_range_fallback(float *d_out, const float *d_x, int S, const KvlMlaConfig *cfg, const KvlMlaBF16 *w) {
    Ctx &c = ctx();
    Dims d;
    if (!dims_of(cfg, d) || !prefill_mfma_shape(d)) return 0;
    int flag = 0;
    HIP_TRY(hipMemcpy(&flag, prefill_range_flag(c.scores.p), sizeof flag, hipMemcpyDeviceToHost));
    if (!flag) return 0;
    if (prefill_device(d_out, d_x, S, cfg, w, nullptr, true, true) != 0) return -1;
    HIP_TRY(hipStreamSynchronize(c.stream));
    return 0;
}

// Causal prefill of seq_len tokens plus the fill of state rows [0, seq_len) from the same x
// (src/generate.c:208-210 calls kvl_mla_prefill_bf16 and then the state prefill on the same
// x). Results equal those two calls; the kv_a projection is computed once where the prefill
// computes it with the decode arithmetic (PrefillKva), else the fill computes its own from
// d_x. Device x and out; host_rows as in fill_rows.
template <class S>
int prefill_state_device(float *d_out, const float *d_x, int seq_len, const KvlMlaConfig *cfg,
                         const KvlMlaBF16 *w, S *s, bool host_rows, bool host_call = false) {
    FillCtx f;
    if (!d_out || !d_x) {
        set_err("invalid arguments");
        return -1;
    }
    if (ctx().capturing) {
        set_err("prefill with state fill during graph capture");
        return -1;
    }
    if (fill_begin(seq_len, cfg, w, s, f) != 0) return -1;
    PrefillKva kv{};
    if (prefill_device(d_out, d_x, seq_len, cfg, w, &kv, host_call) != 0) return -1;
    if (kv.y) {
        if (fill_rows(s, f, kv.y, kv.ldy, kv.np, kv.pstride, 0, seq_len, host_rows) != 0) return -1;
    } else {
        Ctx &c = ctx();
        const int chunk = 4096;
        if (dev_reserve(c.fillx, fill_x_bytes(f.d, std::min(chunk, seq_len))) != 0) return -1;
        for (int t0 = 0; t0 < seq_len; t0 += chunk) {
            const int n = std::min(chunk, seq_len - t0);
            if (fill_from_x(s, f, d_x + (size_t)t0 * f.d.H, c.fillx.p, t0, n, host_rows) != 0) return -1;
        }
    }
    s->len = seq_len;
    f.m->synced = seq_len;
    return 0;
}

template <class S>
int prefill_state(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                  S *s) {
    if (!out || !x || seq_len <= 0 || !cfg || cfg->hidden_size <= 0) {
        set_err("invalid arguments");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    const size_t io = (size_t)seq_len * cfg->hidden_size * sizeof(float);
    const size_t io_al = (io + 255) & ~(size_t)255;
    if (dev_reserve(c.prefill, 2 * io_al) != 0) return -1;
    float *dx = (float *)c.prefill.p;
    float *dout = (float *)((char *)c.prefill.p + io_al);
    HIP_TRY(hipMemcpyAsync(dx, x, io, hipMemcpyHostToDevice, c.stream));
    if (prefill_state_device(dout, dx, seq_len, cfg, w, s, true, true) != 0) return -1;
    HIP_TRY(hipStreamSynchronize(c.stream));
    // the state rows do not depend on the attention; only the output is computed again
    if (prefill_range_fallback(dout, dx, seq_len, cfg, w) != 0) return -1;
    HIP_TRY(hipMemcpyAsync(out, dout, io, hipMemcpyDeviceToHost, c.stream));
    HIP_TRY(hipStreamSynchronize(c.stream));
    return 0;
}

// A captured graph and the free generation at its capture.
struct GraphHandle {
    hipGraphExec_t exec;
    uint64_t gen;
};

struct Guard {
    std::lock_guard<std::recursive_mutex> g;
    Guard() : g(ctx().mu) { g_err.clear(); }
};

}  // namespace

// ==================================================================== C ABI ==============

extern "C" {

// ---- include/kvl/ops.h ---------------------------------------------------------------

// src/ops.c:12-17: the BF16 word is the high half of the FP32 word (a bit operation).
float kvl_bf16_to_f32(uint16_t x) {
    const uint32_t u = (uint32_t)x << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

// src/ops.c:53-66 on the GPU (void return as the reference: failures leave y untouched and
// are reported through kvl_mla_last_error()).
void kvl_matvec_bf16(float *y, const float *x, const uint16_t *w, int in, int out) {
    Guard guard;
    if (!y || !x || !w || in <= 0 || out <= 0) {
        set_err("invalid arguments");
        return;
    }
    if (ensure_ready() != 0) return;
    Ctx &c = ctx();
    const uint16_t *dw = nullptr;
    if (dev_weight(w, (size_t)in * out, &dw) != 0) return;
    Layout L;
    L.take<float>(nullptr, (size_t)in);
    L.take<float>(nullptr, (size_t)out);
    if (dev_reserve(c.prefill, L.off) != 0) return;
    Layout L2;
    float *dx = L2.take<float>((char *)c.prefill.p, (size_t)in);
    float *dy = L2.take<float>((char *)c.prefill.p, (size_t)out);
    if (hipMemcpyAsync(dx, x, (size_t)in * 4, hipMemcpyHostToDevice, c.stream) != hipSuccess ||
        launch_gemv(c.stream, dy, out, dx, in, 1, dw, out, nullptr, 0, in, false) != hipSuccess ||
        hipMemcpyAsync(y, dy, (size_t)out * 4, hipMemcpyDeviceToHost, c.stream) != hipSuccess ||
        hipStreamSynchronize(c.stream) != hipSuccess)
        set_err("kvl_matvec_bf16: device error");
}

// src/ops.c:76-83 on the GPU.
void kvl_rmsnorm_bf16(float *y, const float *x, const uint16_t *weight, int n, float eps) {
    Guard guard;
    if (!y || !x || !weight || n <= 0) {
        set_err("invalid arguments");
        return;
    }
    if (ensure_ready() != 0) return;
    Ctx &c = ctx();
    Layout L;
    L.take<float>(nullptr, (size_t)n);
    L.take<float>(nullptr, (size_t)n);
    L.take<uint16_t>(nullptr, (size_t)n);
    if (dev_reserve(c.prefill, L.off) != 0) return;
    Layout L2;
    char *base = (char *)c.prefill.p;
    float *dx = L2.take<float>(base, (size_t)n);
    float *dy = L2.take<float>(base, (size_t)n);
    uint16_t *dwt = L2.take<uint16_t>(base, (size_t)n);
    if (hipMemcpyAsync(dx, x, (size_t)n * 4, hipMemcpyHostToDevice, c.stream) != hipSuccess ||
        hipMemcpyAsync(dwt, weight, (size_t)n * 2, hipMemcpyHostToDevice, c.stream) != hipSuccess ||
        launch_rmsnorm(c.stream, dy, dx, dwt, n, 1, eps) != hipSuccess ||
        hipMemcpyAsync(y, dy, (size_t)n * 4, hipMemcpyDeviceToHost, c.stream) != hipSuccess ||
        hipStreamSynchronize(c.stream) != hipSuccess)
        set_err("kvl_rmsnorm_bf16: device error");
}

// src/mla_prefill_streaming.c:78-206 (declared at include/kvl/ops.h:63-64), on the GPU.
int kvl_mla_prefill_bf16(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg,
                         const KvlMlaBF16 *w) {
    Guard guard;
    Dims d;
    if (!out || !x || seq_len <= 0 || !weights_ok(w) || !dims_of(cfg, d)) {
        set_err("invalid arguments");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    const size_t io = (size_t)seq_len * d.H * sizeof(float);
    if (dev_reserve(c.prefill, 2 * io + 512) != 0) return -1;
    float *dx = (float *)c.prefill.p;
    float *dout = (float *)((char *)c.prefill.p + ((io + 255) & ~(size_t)255));
    HIP_TRY(hipMemcpyAsync(dx, x, io, hipMemcpyHostToDevice, c.stream));
    if (prefill_device(dout, dx, seq_len, cfg, w, nullptr, true) != 0) return -1;
    HIP_TRY(hipStreamSynchronize(c.stream));
    if (prefill_range_fallback(dout, dx, seq_len, cfg, w) != 0) return -1;
    HIP_TRY(hipMemcpyAsync(out, dout, io, hipMemcpyDeviceToHost, c.stream));
    HIP_TRY(hipStreamSynchronize(c.stream));
    return 0;
}

int kvl_mla_prefill_device(float *d_out, const float *d_x, int seq_len, const KvlMlaConfig *cfg,
                           const KvlMlaBF16 *w) {
    Guard guard;
    return prefill_device(d_out, d_x, seq_len, cfg, w);
}

int kvl_mla_prefill_compressed_state_bf16(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg,
                                          const KvlMlaBF16 *w, KvlMlaCompressedState *state) {
    Guard guard;
    return prefill_state(out, x, seq_len, cfg, w, state);
}

int kvl_mla_prefill_compressed_q8_state_bf16(float *out, const float *x, int seq_len,
                                             const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                             KvlMlaCompressedQ8State *state) {
    Guard guard;
    return prefill_state(out, x, seq_len, cfg, w, state);
}

int kvl_mla_prefill_compressed_state_device(float *d_out, const float *d_x, int seq_len,
                                            const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                            KvlMlaCompressedState *state) {
    Guard guard;
    return prefill_state_device(d_out, d_x, seq_len, cfg, w, state, false);
}

int kvl_mla_prefill_compressed_q8_state_device(float *d_out, const float *d_x, int seq_len,
                                               const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                               KvlMlaCompressedQ8State *state) {
    Guard guard;
    return prefill_state_device(d_out, d_x, seq_len, cfg, w, state, false);
}

int kvl_mla_prefill_compressed_bf16_state_bf16(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg,
                                               const KvlMlaBF16 *w, KvlMlaCompressedBF16State *state) {
    Guard guard;
    return prefill_state(out, x, seq_len, cfg, w, state);
}

int kvl_mla_prefill_compressed_bf16_state_device(float *d_out, const float *d_x, int seq_len,
                                                 const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                                 KvlMlaCompressedBF16State *state) {
    Guard guard;
    return prefill_state_device(d_out, d_x, seq_len, cfg, w, state, false);
}

// ---- include/kvl/mla_state.h (expanded state) ------------------------------------------

int kvl_mla_state_init(KvlMlaState *state, const KvlMlaConfig *cfg, int capacity) {
    Guard guard;
    if (!state || !cfg || capacity <= 0 || cfg->num_heads <= 0 || cfg->qk_nope_dim <= 0 ||
        cfg->qk_rope_dim <= 0 || cfg->v_head_dim <= 0)
        return -1;
    mirror_drop(state);
    memset(state, 0, sizeof(*state));
    const size_t qd = (size_t)cfg->qk_nope_dim + (size_t)cfg->qk_rope_dim;
    state->keys = (float *)calloc((size_t)capacity * cfg->num_heads * qd, sizeof(float));
    state->values =
        (float *)calloc((size_t)capacity * cfg->num_heads * (size_t)cfg->v_head_dim, sizeof(float));
    if (!state->keys || !state->values) {
        free(state->keys);
        free(state->values);
        memset(state, 0, sizeof(*state));
        return -1;
    }
    state->capacity = capacity;
    state->num_heads = cfg->num_heads;
    state->qk_nope_dim = cfg->qk_nope_dim;
    state->qk_rope_dim = cfg->qk_rope_dim;
    state->v_head_dim = cfg->v_head_dim;
    return 0;
}

void kvl_mla_state_reset(KvlMlaState *state) {
    Guard guard;
    if (!state) return;
    state->len = 0;
    mirror_lower(state, 0);
}

void kvl_mla_state_free(KvlMlaState *state) {
    Guard guard;
    if (!state) return;
    mirror_drop(state);
    free(state->keys);
    free(state->values);
    memset(state, 0, sizeof(*state));
}

size_t kvl_mla_state_bytes(const KvlMlaState *state) {
    if (!state || state->capacity <= 0) return 0;
    const size_t qd = (size_t)state->qk_nope_dim + (size_t)state->qk_rope_dim;
    const size_t per = (size_t)state->num_heads * (qd + (size_t)state->v_head_dim) * sizeof(float);
    return sizeof(*state) + (size_t)state->capacity * per;
}

int kvl_mla_decode_bf16(float *out, const float *x, int position, const KvlMlaConfig *cfg,
                        const KvlMlaBF16 *w, KvlMlaState *state) {
    Guard guard;
    KvlMlaState *st[1] = {state};
    return decode_host(out, x, &position, 1, cfg, w, st);
}

// ---- include/kvl/mla_compressed_state.h ---------------------------------------------------

int kvl_mla_compressed_state_init(KvlMlaCompressedState *state, const KvlMlaConfig *cfg, int capacity) {
    Guard guard;
    if (!state || !cfg || capacity <= 0 || cfg->kv_lora_rank <= 0 || cfg->qk_rope_dim <= 0 ||
        (cfg->qk_rope_dim & 1))
        return -1;
    mirror_drop(state);
    memset(state, 0, sizeof(*state));
    state->latent = (float *)calloc((size_t)capacity * cfg->kv_lora_rank, sizeof(float));
    state->rope = (float *)calloc((size_t)capacity * cfg->qk_rope_dim, sizeof(float));
    if (!state->latent || !state->rope) {
        free(state->latent);
        free(state->rope);
        memset(state, 0, sizeof(*state));
        return -1;
    }
    state->capacity = capacity;
    state->kv_lora_rank = cfg->kv_lora_rank;
    state->qk_rope_dim = cfg->qk_rope_dim;
    return 0;
}

void kvl_mla_compressed_state_reset(KvlMlaCompressedState *state) {
    Guard guard;
    if (!state) return;
    state->len = 0;
    mirror_lower(state, 0);
}

int kvl_mla_compressed_state_truncate(KvlMlaCompressedState *state, int new_len) {
    Guard guard;
    if (!state || new_len < 0 || new_len > state->len) return -1;
    state->len = new_len;
    mirror_lower(state, new_len);
    return 0;
}

void kvl_mla_compressed_state_free(KvlMlaCompressedState *state) {
    Guard guard;
    if (!state) return;
    mirror_drop(state);
    free(state->latent);
    free(state->rope);
    memset(state, 0, sizeof(*state));
}

size_t kvl_mla_compressed_state_bytes(const KvlMlaCompressedState *state) {
    if (!state || state->capacity <= 0) return 0;
    return sizeof(*state) + (size_t)state->capacity *
                                ((size_t)state->kv_lora_rank + (size_t)state->qk_rope_dim) * sizeof(float);
}

int kvl_mla_compressed_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                          const KvlMlaBF16 *w, KvlMlaCompressedState *state) {
    Guard guard;
    return state_prefill(x, seq_len, cfg, w, state);
}

int kvl_mla_decode_compressed_bf16(float *out, const float *x, int position, const KvlMlaConfig *cfg,
                                   const KvlMlaBF16 *w, KvlMlaCompressedState *state) {
    Guard guard;
    KvlMlaCompressedState *st[1] = {state};
    return decode_host(out, x, &position, 1, cfg, w, st);
}

// src/mla_compressed_state.c:163-184: every token of the block takes the single-token path,
// so block and serial decode agree exactly.
int kvl_mla_decode_compressed_block_bf16(float *out, const float *x, int count, int start_position,
                                         const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                         KvlMlaCompressedState *state) {
    Guard guard;
    return decode_block(out, x, count, start_position, cfg, w, state);
}

int kvl_mla_decode_compressed_q8_block_bf16(float *out, const float *x, int count, int start_position,
                                            const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                            KvlMlaCompressedQ8State *state) {
    Guard guard;
    return decode_block(out, x, count, start_position, cfg, w, state);
}

// ---- BF16-latent state (include/kvl/mla_hip.h) -------------------------------------------
// The FP32 state's life cycle and checks (src/mla_compressed_state.c:24-50) over bf16 arrays.

int kvl_mla_compressed_bf16_state_init(KvlMlaCompressedBF16State *state, const KvlMlaConfig *cfg, int capacity) {
    Guard guard;
    if (!state || !cfg || capacity <= 0 || cfg->kv_lora_rank <= 0 || cfg->qk_rope_dim <= 0 ||
        (cfg->qk_rope_dim & 1)) {
        set_err("invalid arguments");
        return -1;
    }
    mirror_drop(state);
    memset(state, 0, sizeof(*state));
    state->latent = (uint16_t *)calloc((size_t)capacity * cfg->kv_lora_rank, sizeof(uint16_t));
    state->rope = (uint16_t *)calloc((size_t)capacity * cfg->qk_rope_dim, sizeof(uint16_t));
    if (!state->latent || !state->rope) {
        free(state->latent);
        free(state->rope);
        memset(state, 0, sizeof(*state));
        set_err("host allocation of %d rows failed", capacity);
        return -1;
    }
    state->capacity = capacity;
    state->kv_lora_rank = cfg->kv_lora_rank;
    state->qk_rope_dim = cfg->qk_rope_dim;
    return 0;
}

void kvl_mla_compressed_bf16_state_reset(KvlMlaCompressedBF16State *state) {
    Guard guard;
    if (!state) return;
    state->len = 0;
    mirror_lower(state, 0);
}

int kvl_mla_compressed_bf16_state_truncate(KvlMlaCompressedBF16State *state, int new_len) {
    Guard guard;
    if (!state || new_len < 0 || new_len > state->len) {
        set_err("invalid truncate length");
        return -1;
    }
    state->len = new_len;
    mirror_lower(state, new_len);
    return 0;
}

void kvl_mla_compressed_bf16_state_free(KvlMlaCompressedBF16State *state) {
    Guard guard;
    if (!state) return;
    mirror_drop(state);
    free(state->latent);
    free(state->rope);
    memset(state, 0, sizeof(*state));
}

size_t kvl_mla_compressed_bf16_state_bytes(const KvlMlaCompressedBF16State *state) {
    if (!state || state->capacity <= 0) return 0;
    return sizeof(*state) + (size_t)state->capacity *
                                ((size_t)state->kv_lora_rank + (size_t)state->qk_rope_dim) * sizeof(uint16_t);
}

int kvl_mla_compressed_bf16_state_sync(KvlMlaCompressedBF16State *state) {
    Guard guard;
    if (!state) return -1;
    mirror_lower(state, 0);
    return 0;
}

int kvl_mla_compressed_bf16_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                               const KvlMlaBF16 *w, KvlMlaCompressedBF16State *state) {
    Guard guard;
    return state_prefill(x, seq_len, cfg, w, state);
}

int kvl_mla_decode_compressed_bf16_bf16(float *out, const float *x, int position, const KvlMlaConfig *cfg,
                                        const KvlMlaBF16 *w, KvlMlaCompressedBF16State *state) {
    Guard guard;
    KvlMlaCompressedBF16State *st[1] = {state};
    return decode_host(out, x, &position, 1, cfg, w, st);
}

int kvl_mla_decode_compressed_bf16_block_bf16(float *out, const float *x, int count, int start_position,
                                              const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                              KvlMlaCompressedBF16State *state) {
    Guard guard;
    return decode_block(out, x, count, start_position, cfg, w, state);
}

int kvl_mla_decode_compressed_bf16_batch_bf16(float *out, const float *x, const int *positions, int batch,
                                              const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                              KvlMlaCompressedBF16State *const *states) {
    Guard guard;
    if (!positions) {
        set_err("invalid arguments");
        return -1;
    }
    return decode_host(out, x, positions, batch, cfg, w, states);
}

int kvl_mla_decode_compressed_bf16_batch_device(float *d_out, const float *d_x, int batch,
                                                const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                                KvlMlaCompressedBF16State *const *states, unsigned flags) {
    Guard guard;
    return decode_device(d_out, d_x, batch, cfg, w, states, flags);
}

// ---- include/kvl/mla_compressed_q8_state.h ----------------------------------------------

int kvl_mla_compressed_q8_state_init(KvlMlaCompressedQ8State *state, const KvlMlaConfig *cfg,
                                     int capacity) {
    Guard guard;
    if (!state || !cfg || capacity <= 0 || cfg->kv_lora_rank <= 0 || cfg->qk_rope_dim <= 0 ||
        (cfg->qk_rope_dim & 1))
        return -1;
    mirror_drop(state);
    memset(state, 0, sizeof(*state));
    state->latent_q8 = (int8_t *)calloc((size_t)capacity * cfg->kv_lora_rank, 1);
    state->latent_scale = (float *)calloc((size_t)capacity, sizeof(float));
    state->rope_bf16 = (uint16_t *)calloc((size_t)capacity * cfg->qk_rope_dim, sizeof(uint16_t));
    if (!state->latent_q8 || !state->latent_scale || !state->rope_bf16) {
        free(state->latent_q8);
        free(state->latent_scale);
        free(state->rope_bf16);
        memset(state, 0, sizeof(*state));
        return -1;
    }
    state->capacity = capacity;
    state->kv_lora_rank = cfg->kv_lora_rank;
    state->qk_rope_dim = cfg->qk_rope_dim;
    return 0;
}

void kvl_mla_compressed_q8_state_reset(KvlMlaCompressedQ8State *state) {
    Guard guard;
    if (!state) return;
    state->len = 0;
    mirror_lower(state, 0);
}

int kvl_mla_compressed_q8_state_truncate(KvlMlaCompressedQ8State *state, int new_len) {
    Guard guard;
    if (!state || new_len < 0 || new_len > state->len) return -1;
    state->len = new_len;
    mirror_lower(state, new_len);
    return 0;
}

void kvl_mla_compressed_q8_state_free(KvlMlaCompressedQ8State *state) {
    Guard guard;
    if (!state) return;
    mirror_drop(state);
    free(state->latent_q8);
    free(state->latent_scale);
    free(state->rope_bf16);
    memset(state, 0, sizeof(*state));
}

size_t kvl_mla_compressed_q8_state_bytes(const KvlMlaCompressedQ8State *state) {
    if (!state || state->capacity <= 0) return 0;
    return sizeof(*state) + (size_t)state->capacity * ((size_t)state->kv_lora_rank + sizeof(float) +
                                                       (size_t)state->qk_rope_dim * sizeof(uint16_t));
}

int kvl_mla_compressed_q8_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                             const KvlMlaBF16 *w, KvlMlaCompressedQ8State *state) {
    Guard guard;
    return state_prefill(x, seq_len, cfg, w, state);
}

int kvl_mla_decode_compressed_q8_bf16(float *out, const float *x, int position,
                                      const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                      KvlMlaCompressedQ8State *state) {
    Guard guard;
    KvlMlaCompressedQ8State *st[1] = {state};
    return decode_host(out, x, &position, 1, cfg, w, st);
}

// ---- include/kvl/mla_hip.h ----------------------------------------------------------------

const char *kvl_mla_last_error(void) { return g_err.c_str(); }

int kvl_mla_init(void) {
    Guard guard;
    return ensure_ready();
}

int kvl_mla_bind_weights(const KvlMlaConfig *cfg, const KvlMlaBF16 *w) {
    Guard guard;
    Dims d;
    if (!weights_ok(w) || !dims_of(cfg, d)) {
        set_err("invalid arguments");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    DevWeights dw;
    if (dev_weights(w, d, dw) != 0) return -1;
    const void *ptrs[5] = {w->q_proj, w->kv_a_proj, w->kv_a_norm, w->kv_b_proj, w->o_proj};
    for (const void *p : ptrs) ctx().weights[p].pins += 1;
    return 0;
}

int kvl_mla_release_weights(const KvlMlaBF16 *w) {
    Guard guard;
    if (!weights_ok(w)) return -1;
    Ctx &c = ctx();
    const void *ptrs[5] = {w->q_proj, w->kv_a_proj, w->kv_a_norm, w->kv_b_proj, w->o_proj};
    for (const void *p : ptrs) {
        auto it = c.weights.find(p);
        if (it == c.weights.end()) continue;
        if (it->second.pins > 0) it->second.pins -= 1;
        if (it->second.pins == 0) {
            (void)dev_free(it->second.dev);
            if (it->second.dev16) (void)dev_free(it->second.dev16);
            if (it->second.devt) (void)dev_free(it->second.devt);
            c.weights.erase(it);
        }
    }
    return 0;
}

int kvl_mla_compressed_state_sync(KvlMlaCompressedState *state) {
    Guard guard;
    if (!state) return -1;
    mirror_lower(state, 0);
    return 0;
}
int kvl_mla_compressed_q8_state_sync(KvlMlaCompressedQ8State *state) {
    Guard guard;
    if (!state) return -1;
    mirror_lower(state, 0);
    return 0;
}
int kvl_mla_state_sync(KvlMlaState *state) {
    Guard guard;
    if (!state) return -1;
    mirror_lower(state, 0);
    return 0;
}

int kvl_mla_decode_compressed_batch_bf16(float *out, const float *x, const int *positions, int batch,
                                         const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                         KvlMlaCompressedState *const *states) {
    Guard guard;
    if (!positions) return -1;
    return decode_host(out, x, positions, batch, cfg, w, states);
}

int kvl_mla_decode_compressed_q8_batch_bf16(float *out, const float *x, const int *positions,
                                            int batch, const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                            KvlMlaCompressedQ8State *const *states) {
    Guard guard;
    if (!positions) return -1;
    return decode_host(out, x, positions, batch, cfg, w, states);
}

int kvl_mla_decode_compressed_q8_batch_device(float *d_out, const float *d_x, int batch,
                                              const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                              KvlMlaCompressedQ8State *const *states, unsigned flags) {
    Guard guard;
    return decode_device(d_out, d_x, batch, cfg, w, states, flags);
}

int kvl_mla_decode_compressed_q8_batch_device_noalloc(float *d_out, const float *d_x, int batch,
                                                      const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                                      KvlMlaCompressedQ8State *const *states, unsigned flags) {
    Guard guard;
    return decode_q8_noalloc(d_out, d_x, batch, cfg, w, states, flags);
}

int kvl_mla_decode_compressed_batch_device(float *d_out, const float *d_x, int batch,
                                           const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                           KvlMlaCompressedState *const *states, unsigned flags) {
    Guard guard;
    return decode_device(d_out, d_x, batch, cfg, w, states, flags);
}

int kvl_mla_attention_layer_q8_device(float *d_h, float *d_n2, int batch, const KvlMlaConfig *cfg,
                                      const KvlMlaBF16 *w, const uint16_t *input_norm,
                                      const uint16_t *post_attn_norm,
                                      KvlMlaCompressedQ8State *const *states, unsigned flags) {
    Guard guard;
    return attention_layer_device(d_h, d_n2, batch, cfg, w, input_norm, post_attn_norm, states, flags);
}

int kvl_mla_attention_layer_device(float *d_h, float *d_n2, int batch, const KvlMlaConfig *cfg,
                                   const KvlMlaBF16 *w, const uint16_t *input_norm,
                                   const uint16_t *post_attn_norm, KvlMlaCompressedState *const *states,
                                   unsigned flags) {
    Guard guard;
    return attention_layer_device(d_h, d_n2, batch, cfg, w, input_norm, post_attn_norm, states, flags);
}

int kvl_mla_attention_layer_bf16_device(float *d_h, float *d_n2, int batch, const KvlMlaConfig *cfg,
                                        const KvlMlaBF16 *w, const uint16_t *input_norm,
                                        const uint16_t *post_attn_norm,
                                        KvlMlaCompressedBF16State *const *states, unsigned flags) {
    Guard guard;
    return attention_layer_device(d_h, d_n2, batch, cfg, w, input_norm, post_attn_norm, states, flags);
}

void *kvl_mla_stream(void) {
    Guard guard;
    if (ensure_ready() != 0) return nullptr;
    return (void *)ctx().stream;
}

int kvl_mla_synchronize(void) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    HIP_TRY(hipStreamSynchronize(c.stream));
    if (*c.fq_err) {  // a stream-ordered fused decode since the last check had a wait time out
        *c.fq_err = 0;
        c.fq_dirty = true;
        set_err("a wait of a fused decode launch timed out (its results are invalid); "
                "KVL_MLA_NO_FUSED_QPREP=1 selects the two-launch form");
        return -1;
    }
    return 0;
}

int kvl_mla_prefill_range_status(void) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    if (c.capturing) {
        set_err("range status during graph capture");
        return -1;
    }
    HIP_TRY(hipStreamSynchronize(c.stream));
    if (!c.rflag.p) return 0;
    int flag = 0;
    HIP_TRY(hipMemcpy(&flag, c.rflag.p, sizeof flag, hipMemcpyDeviceToHost));
    if (flag) {
        HIP_TRY(hipMemset(c.rflag.p, 0, sizeof flag));
        set_err("a stream-ordered prefill met query rows outside the MFMA route's range (row max logit beyond "
                "512 or non-finite operands); its output was written as NaN");
    }
    return flag ? 1 : 0;
}

void *kvl_mla_device_alloc(size_t bytes) {
    Guard guard;
    if (ensure_ready() != 0) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        set_err("hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int kvl_mla_device_free(void *p) {
    Guard guard;
    if (!p) return 0;
    HIP_TRY(hipFree(p));
    return 0;
}

int kvl_mla_copy_to_device(void *dst, const void *src, size_t bytes) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx().stream));
    HIP_TRY(hipStreamSynchronize(ctx().stream));
    return 0;
}

int kvl_mla_copy_to_host(void *dst, const void *src, size_t bytes) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx().stream));
    HIP_TRY(hipStreamSynchronize(ctx().stream));
    return 0;
}

int kvl_mla_capture_begin(void) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    HIP_TRY(hipStreamBeginCapture(ctx().stream, hipStreamCaptureModeThreadLocal));
    ctx().capturing = true;
    return 0;
}

int kvl_mla_capture_end(void **graph_exec) {
    Guard guard;
    Ctx &c = ctx();
    if (!c.capturing || !graph_exec) return -1;
    c.capturing = false;
    hipGraph_t graph = nullptr;
    HIP_TRY(hipStreamEndCapture(c.stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
        set_err("hipGraphInstantiate: %s", hipGetErrorString(e));
        return -1;
    }
    *graph_exec = (void *)new GraphHandle{exec, c.free_gen};
    return 0;
}

int kvl_mla_graph_launch(void *graph_exec) {
    Guard guard;
    if (!graph_exec) return -1;
    const GraphHandle *g = (const GraphHandle *)graph_exec;
    if (g->gen != ctx().free_gen) {
        set_err("library device memory was released or reallocated after this graph was captured "
                "(workspace or RoPE table growth, state free/re-init, weight release): capture it again");
        return -1;
    }
    Ctx &c = ctx();
    if (c.fq_dirty && c.fq_flags) {  // a graph's fused launches expect clean flags
        HIP_TRY(launch_clear_flags(c.stream, c.fq_flags, kFqFlagLines));
        c.fq_dirty = false;
    }
    HIP_TRY(hipGraphLaunch(g->exec, c.stream));
    return 0;
}

int kvl_mla_graph_destroy(void *graph_exec) {
    Guard guard;
    if (!graph_exec) return 0;
    GraphHandle *g = (GraphHandle *)graph_exec;
    const hipError_t e = hipGraphExecDestroy(g->exec);
    delete g;
    HIP_TRY(e);
    return 0;
}

int kvl_mla_q8_pack_rows(int8_t *codes, float *scales, uint16_t *rope_bf16, const float *latent,
                         const float *k_rope_raw, const int *positions, int n, int R, int DR,
                         float theta) {
    Guard guard;
    if (!codes || !scales || !rope_bf16 || !latent || !k_rope_raw || !positions || n <= 0 || R <= 0 ||
        R > 1024 || DR <= 0 || DR > 256 || (DR & 1) || !(theta > 0.0f)) {
        set_err("invalid arguments");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    int maxpos = 0;
    for (int i = 0; i < n; ++i) {
        if (positions[i] < 0) {
            set_err("negative position");
            return -1;
        }
        maxpos = std::max(maxpos, positions[i]);
    }
    const float2 *cs = nullptr;
    if (rope_table(theta, DR, maxpos + 1, &cs) != 0) return -1;
    const size_t rb = row_bytes_of(kFmtQ8, R, DR, 0);
    const int KVO = R + DR;
    // device: input rows [n, R+DR], scratch history (codes/scales/rope) [n], staged rows
    Layout L;
    L.take<float>(nullptr, (size_t)n * KVO);
    L.take<int8_t>(nullptr, (size_t)n * R);
    L.take<float>(nullptr, (size_t)n);
    L.take<uint16_t>(nullptr, (size_t)n * DR);
    L.take<uint8_t>(nullptr, (size_t)n * rb);
    if (dev_reserve(c.prefill, L.off) != 0) return -1;
    Layout L2;
    char *base = (char *)c.prefill.p;
    float *din = L2.take<float>(base, (size_t)n * KVO);
    int8_t *dcodes = L2.take<int8_t>(base, (size_t)n * R);
    float *dscl = L2.take<float>(base, (size_t)n);
    uint16_t *drope = L2.take<uint16_t>(base, (size_t)n * DR);
    uint8_t *drows = L2.take<uint8_t>(base, (size_t)n * rb);
    std::vector<float> hin((size_t)n * KVO);
    for (int i = 0; i < n; ++i) {
        memcpy(&hin[(size_t)i * KVO], latent + (size_t)i * R, (size_t)R * 4);
        memcpy(&hin[(size_t)i * KVO + R], k_rope_raw + (size_t)i * DR, (size_t)DR * 4);
    }
    HIP_TRY(hipMemcpyAsync(din, hin.data(), hin.size() * 4, hipMemcpyHostToDevice, c.stream));
    Dims d{};
    d.R = R;
    d.DR = DR;
    d.NH = 1;
    // one block per row, each row its own one-row "sequence" at its own position
    for (int g0 = 0; g0 < n; g0 += kMaxBatch) {
        const int m = std::min(kMaxBatch, n - g0);
        SeqTable t;
        memset(&t, 0, sizeof t);
        t.n = m;
        for (int i = 0; i < m; ++i) {
            // row g0+i of the scratch history is written at "position" positions[g0+i]; point
            // the arrays so that row pos lands on scratch row g0+i.
            const long off = (long)(g0 + i) - (long)positions[g0 + i];
            t.s[i].a = dcodes + off * R;
            t.s[i].b = dscl + off;
            t.s[i].c = drope + off * DR;
            t.s[i].pos = positions[g0 + i];
        }
        DecodeWork wk{};
        wk.rows = drows + (size_t)g0 * rb;
        HIP_TRY(launch_append(c.stream, kFmtQ8, t, d, din + (size_t)g0 * KVO, KVO, 0, 1, 0, nullptr, 0.f, cs,
                              wk, true, 0));
    }
    std::vector<uint8_t> hrows((size_t)n * rb);
    HIP_TRY(hipMemcpyAsync(hrows.data(), drows, hrows.size(), hipMemcpyDeviceToHost, c.stream));
    HIP_TRY(hipStreamSynchronize(c.stream));
    for (int i = 0; i < n; ++i) {
        const uint8_t *row = &hrows[(size_t)i * rb];
        memcpy(codes + (size_t)i * R, row, (size_t)R);
        memcpy(scales + i, row + R, 4);
        memcpy(rope_bf16 + (size_t)i * DR, row + R + 4, 2 * (size_t)DR);
    }
    return 0;
}

int kvl_mla_timing_enable(int on) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    if (on < 0 || on > 2) return -1;
    ctx().timing = on != 0;
    ctx().timing_graph = on == 2;
    return 0;
}

int kvl_mla_set_fused_qprep(int on) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    if (on != 0 && on != 1) {
        set_err("kvl_mla_set_fused_qprep: on must be 0 or 1");
        return -1;
    }
    const int prev = ctx().fq_on ? 1 : 0;
    ctx().fq_on = on == 1;
    return prev;
}

int kvl_mla_set_fused_combine(int on) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    if (on != 0 && on != 1) {
        set_err("kvl_mla_set_fused_combine: on must be 0 or 1");
        return -1;
    }
    const int prev = ctx().comb_on ? 1 : 0;
    ctx().comb_on = on == 1;
    return prev;
}

int kvl_mla_set_fused_projection(int on) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    if (on != 0 && on != 1) {
        set_err("kvl_mla_set_fused_projection: on must be 0 or 1");
        return -1;
    }
    const int prev = ctx().gemv_on ? 1 : 0;
    ctx().gemv_on = on == 1;
    return prev;
}

int kvl_mla_set_fused_wait_limit(unsigned ticks) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    ctx().fq_spin = ticks == 0 ? kFqSpinTicks : ticks;
    return 0;
}

int kvl_mla_timing_stages(unsigned mask) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    ctx().timing_mask = mask & ((1u << kStages) - 1);
    return 0;
}

// Sums the recorded stage durations (ms) into ms[0..5] and launch counts into count[0..5]
// (gemv_in, append, qprep, attention, combine, gemv_out), then clears the records.
int kvl_mla_timing_read(double *ms, int *count) {
    Guard guard;
    Ctx &c = ctx();
    if (!ms || !count) return -1;
    for (int i = 0; i < kStages; ++i) {
        ms[i] = 0.0;
        count[i] = 0;
    }
    int rc = 0;
    for (auto &u : c.ev_used) {
        float t = 0.f;
        if (hipEventSynchronize(u.second.second) != hipSuccess ||
            hipEventElapsedTime(&t, u.second.first, u.second.second) != hipSuccess) {
            set_err("event timing failed");
            rc = -1;
        } else if (u.first >= 0 && u.first < kStages) {
            ms[u.first] += t;
            count[u.first] += 1;
        }
        c.ev_pool.push_back(u.second.first);
        c.ev_pool.push_back(u.second.second);
    }
    c.ev_used.clear();
    return rc;
}

void *kvl_mla_event_record(void) {
    Guard guard;
    if (ensure_ready() != 0) return nullptr;
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess || hipEventRecord(e, ctx().stream) != hipSuccess) {
        set_err("event record failed");
        return nullptr;
    }
    return (void *)e;
}

double kvl_mla_event_elapsed_ms(void *start, void *end) {
    Guard guard;
    float t = -1.f;
    if (!start || !end || hipEventSynchronize((hipEvent_t)end) != hipSuccess ||
        hipEventElapsedTime(&t, (hipEvent_t)start, (hipEvent_t)end) != hipSuccess) {
        set_err("event elapsed failed");
        return -1.0;
    }
    return (double)t;
}

int kvl_mla_event_destroy(void *ev) {
    Guard guard;
    if (ev) HIP_TRY(hipEventDestroy((hipEvent_t)ev));
    return 0;
}

int kvl_mla_copy_kernel(void *dst, const void *src, size_t bytes) {
    Guard guard;
    if (!dst || !src || (bytes % 16) != 0) {
        set_err("copy: 16-byte multiple required");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    HIP_TRY(launch_copy(ctx().stream, dst, src, bytes));
    return 0;
}

int kvl_mla_empty_kernel(void) {
    Guard guard;
    if (ensure_ready() != 0) return -1;
    HIP_TRY(launch_empty(ctx().stream));
    return 0;
}

int kvl_mla_read_kernel(const void *src, size_t bytes) {
    Guard guard;
    if (!src || bytes % 16 != 0 || ((uintptr_t)src % 16) != 0) {
        set_err("invalid arguments (16-byte aligned source, bytes %% 16 == 0)");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    if (c.sink.bytes < (size_t)kReadBlocks * 256 * 16) {
        if (c.capturing) {
            set_err("sink allocation during graph capture");
            return -1;
        }
        if (dev_reserve(c.sink, (size_t)kReadBlocks * 256 * 16) != 0) return -1;
    }
    HIP_TRY(launch_read(c.stream, src, bytes, c.sink.p));
    return 0;
}

static int fill_synth(const void *key, const HostView &v, int row0, int nrows, uint64_t seed,
                      void (*set_len)(const void *, int)) {
    if (row0 < 0 || nrows <= 0 || row0 + nrows > v.capacity || row0 > v.len) {
        set_err("invalid row range");
        return -1;
    }
    if (ensure_ready() != 0) return -1;
    Ctx &c = ctx();
    Mirror *m = nullptr;
    if (mirror_get(key, v, &m, true) != 0) return -1;
    if (m->synced < row0 && upload_rows(*m, v, m->synced, row0, c.stream) != 0) return -1;
    HIP_TRY(launch_fill_history(c.stream, v.fmt, m->a, m->b, m->c, v.d0, v.d1, row0, nrows, seed));
    HIP_TRY(hipStreamSynchronize(c.stream));
    m->synced = row0 + nrows;
    set_len(key, row0 + nrows);
    return 0;
}

int kvl_mla_compressed_q8_state_fill_synthetic(KvlMlaCompressedQ8State *state, int row0, int nrows,
                                               uint64_t seed) {
    Guard guard;
    if (!state) return -1;
    return fill_synth(state, view_of(state), row0, nrows, seed,
                      [](const void *k, int len) { ((KvlMlaCompressedQ8State *)k)->len = len; });
}

int kvl_mla_compressed_state_fill_synthetic(KvlMlaCompressedState *state, int row0, int nrows,
                                            uint64_t seed) {
    Guard guard;
    if (!state) return -1;
    return fill_synth(state, view_of(state), row0, nrows, seed,
                      [](const void *k, int len) { ((KvlMlaCompressedState *)k)->len = len; });
}

static int pull_rows(const void *key, const HostView &v, int row0, int nrows) {
    Ctx &c = ctx();
    auto it = c.mirrors.find(key);
    if (it == c.mirrors.end() || row0 < 0 || nrows <= 0 || row0 + nrows > it->second.synced) {
        set_err("rows not on the device");
        return -1;
    }
    Mirror &m = it->second;
    size_t ea, eb, ec;
    comp_bytes(m.fmt, m.d0, m.d1, m.d2, ea, eb, ec);
    HIP_TRY(hipMemcpyAsync((char *)v.ha + ea * row0, (char *)m.a + ea * row0, ea * nrows,
                           hipMemcpyDeviceToHost, c.stream));
    HIP_TRY(hipMemcpyAsync((char *)v.hb + eb * row0, (char *)m.b + eb * row0, eb * nrows,
                           hipMemcpyDeviceToHost, c.stream));
    if (ec)
        HIP_TRY(hipMemcpyAsync((char *)v.hc + ec * row0, (char *)m.c + ec * row0, ec * nrows,
                               hipMemcpyDeviceToHost, c.stream));
    HIP_TRY(hipStreamSynchronize(c.stream));
    return 0;
}

int kvl_mla_compressed_q8_state_pull(KvlMlaCompressedQ8State *state, int row0, int nrows) {
    Guard guard;
    if (!state) return -1;
    return pull_rows(state, view_of(state), row0, nrows);
}

int kvl_mla_compressed_state_pull(KvlMlaCompressedState *state, int row0, int nrows) {
    Guard guard;
    if (!state) return -1;
    return pull_rows(state, view_of(state), row0, nrows);
}

int kvl_mla_compressed_bf16_state_fill_synthetic(KvlMlaCompressedBF16State *state, int row0, int nrows,
                                                 uint64_t seed) {
    Guard guard;
    if (!state) return -1;
    return fill_synth(state, view_of(state), row0, nrows, seed,
                      [](const void *k, int len) { ((KvlMlaCompressedBF16State *)k)->len = len; });
}

int kvl_mla_compressed_bf16_state_pull(KvlMlaCompressedBF16State *state, int row0, int nrows) {
    Guard guard;
    if (!state) return -1;
    return pull_rows(state, view_of(state), row0, nrows);
}

}  // extern "C"
