// slha_abi.cpp — the C ABI of libslha.so (include/slha.h + include/slha_gpu.h).
//
// Boundary semantics follow slha-c/src/lib.rs:
//   * every call clears the thread-local last error and runs under a panic
//     barrier (C++ exceptions -> SLHA_ERR_PANIC, lib.rs:91-105);
//   * outputs are written only after every check passed;
//   * model handles are opaque tokens in a process-wide registry; released
//     tokens are quarantined so a stale pointer never aliases a live model
//     (lib.rs:124-205).
// All compute runs on the GPU: host-pointer entry points stage their buffers
// through per-thread device memory on a per-thread stream.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/slha.h"
#include "../../include/slha_ccos.h"
#include "../../include/slha_eventlog.h"
#include "../../include/slha_gpu.h"
#include "slha_launch.h"

using namespace slha;

namespace {

// ---------------------------------------------------------------------------
// Errors (lib.rs:35-105)

constexpr size_t kErrCap = 512;
thread_local char g_last_error[kErrCap] = {0};

void clear_error() { g_last_error[0] = 0; }

void set_error(const std::string& m) {
    const size_t n = m.size() < kErrCap - 1 ? m.size() : kErrCap - 1;
    std::memcpy(g_last_error, m.data(), n);
    g_last_error[n] = 0;
}

struct SlhaError {
    int32_t code;
    std::string msg;
};

[[noreturn]] void fail(int32_t code, const char* fmt, ...) {
    char buf[kErrCap];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw SlhaError{code, buf};
}

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(SLHA_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

template <class F>
int32_t ffi_status(F&& body) {
    clear_error();
    try {
        body();
        return SLHA_OK;
    } catch (const SlhaError& e) {
        set_error(e.msg);
        return e.code;
    } catch (...) {
        set_error("panic caught at the SLHA C ABI boundary");
        return SLHA_ERR_PANIC;
    }
}

// ---------------------------------------------------------------------------
// Context (lib.rs:107-122, 331-360)

struct ContextObj {
    uint32_t abi_version;
    uint32_t reserved;
};
ContextObj g_context = {SLHA_ABI_VERSION, 0};

// ---------------------------------------------------------------------------
// Product-side SplitMix64 / Box–Muller generator (rng.rs:7-52) for Z and the
// RHT diagonal of head_dim-128 models.

struct Rng {
    uint64_t state;
    explicit Rng(uint64_t seed) : state(seed ^ 0x9E3779B97F4A7C15ull) {}
    uint64_t next_u64() {
        state += 0x9E3779B97F4A7C15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float next_unit() { return (float)(next_u64() >> 40) * (1.0f / 16777216.0f); }
    float next_gaussian() {
        const float u1 = std::fmax(next_unit(), 1.0e-7f);
        const float u2 = next_unit();
        const float r = std::sqrt(-2.0f * std::log(u1));
        return r * std::cos(2.0f * 3.14159265358979323846f * u2);
    }
};

const float kPi = 3.14159265358979323846f;
float lambda_c() { return std::sqrt(kPi / (2.0f * 256.0f)); }  // scenario.rs:30-32
float rht_inv() { return 1.0f / std::sqrt(128.0f); }            // incoherence.rs:66
float sqrt_half_pi() { return std::sqrt(kPi / 2.0f); }          // learned.rs:303

// ---------------------------------------------------------------------------
// Models

// Device copies of a model's projection on one device.
struct DeviceProjection {
    const float* z = nullptr;     // [256][d_pad] f32
    const float* diag = nullptr;  // [d_pad] +-1, or null without RHT
    const void* zpack = nullptr;  // head_dim-128 models: kZPackBytes, MFMA operand pack of Z
    float cert_scale = 0.0f;      // build_projection_pack's scale
    const float* p = nullptr;     // learned models: [128][d]
    const float* p4 = nullptr;    // learned models: P interleaved by 4 columns, [ceil(d/4)][128][4]
    const float* z4 = nullptr;    // learned models: Z interleaved by 4 columns, [ceil(d_pad/4)][256][4]
};

// [R][n] row-major -> interleaved by 4 columns: element (r, i) at
// ((i / 4) * R + r) * 4 + i % 4, zero past n (the layout of the learned
// kernels' row dot products, one contiguous float4 per row and column group).
static void interleave4(const float* m, size_t rows, size_t n, float* out) {
    const size_t groups = (n + 3) / 4;
    std::memset(out, 0, groups * rows * 4 * sizeof(float));
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < n; ++i) out[((i / 4) * rows + r) * 4 + (i % 4)] = m[r * n + i];
}

// A head_dim-128 model (d = d_pad = 128, identity latent, Z [256][128]) or a
// learned model loaded from a .slhw file (d > 128, P [128][d], Z [256][d_pad]).
struct Model {
    size_t d = 128;
    size_t d_pad = 128;
    bool learned = false;
    uint64_t seed = 0;
    bool rht = false;
    int residual_mode = kResidualR;
    std::vector<float> p;     // learned: [128][d]
    std::vector<float> z;     // [256][d_pad]
    std::vector<float> diag;  // [d_pad], +-1
    std::mutex mu;
    std::unordered_map<int, std::pair<DeviceProjection, void*>> dev;  // (views, allocation)

    ~Model() {
        for (auto& kv : dev) {
            int cur = 0;
            if (hipGetDevice(&cur) == hipSuccess && hipSetDevice(kv.first) == hipSuccess) {
                (void)hipFree(kv.second.second);
                (void)hipSetDevice(cur);
            }
        }
    }

    // Z, its MFMA pack and the RHT diagonal on the current device, in one
    // allocation made on first use.
    DeviceProjection device_buffers() {
        int device = 0;
        check_hip(hipGetDevice(&device), "hipGetDevice");
        std::lock_guard<std::mutex> lock(mu);
        auto it = dev.find(device);
        if (it == dev.end()) {
            // [Z][Z pack (head_dim-128 only)][diag][P, P4, Z4 (learned only)], 256-B
            // aligned parts
            const size_t zb = align_up(z.size() * sizeof(float));
            const size_t pkb = learned ? 0 : kZPackBytes;
            const size_t db = align_up(d_pad * sizeof(float));
            const size_t pb = align_up(p.size() * sizeof(float));
            const size_t p4b = learned ? align_up((d + 3) / 4 * 128 * 4 * sizeof(float)) : 0;
            const size_t z4b = learned ? align_up((d_pad + 3) / 4 * 256 * 4 * sizeof(float)) : 0;
            std::vector<char> host(zb + pkb + db + pb + p4b + z4b, 0);
            std::memcpy(host.data(), z.data(), z.size() * sizeof(float));
            DeviceProjection dp;
            if (!learned) dp.cert_scale = build_projection_pack(z.data(), host.data() + zb);
            if (rht) std::memcpy(host.data() + zb + pkb, diag.data(), d_pad * sizeof(float));
            if (learned) {
                char* lp = host.data() + zb + pkb + db;
                std::memcpy(lp, p.data(), p.size() * sizeof(float));
                interleave4(p.data(), 128, d, reinterpret_cast<float*>(lp + pb));
                interleave4(z.data(), 256, d_pad, reinterpret_cast<float*>(lp + pb + p4b));
            }
            char* buf = nullptr;
            check_hip(hipMalloc(&buf, host.size()), "hipMalloc(projection)");
            check_hip(hipMemcpy(buf, host.data(), host.size(), hipMemcpyHostToDevice),
                      "hipMemcpy(projection)");
            dp.z = reinterpret_cast<const float*>(buf);
            dp.zpack = learned ? nullptr : buf + zb;
            dp.diag = rht ? reinterpret_cast<const float*>(buf + zb + pkb) : nullptr;
            dp.p = learned ? reinterpret_cast<const float*>(buf + zb + pkb + db) : nullptr;
            dp.p4 = learned ? reinterpret_cast<const float*>(buf + zb + pkb + db + pb) : nullptr;
            dp.z4 = learned ? reinterpret_cast<const float*>(buf + zb + pkb + db + pb + p4b) : nullptr;
            it = dev.emplace(device, std::make_pair(dp, static_cast<void*>(buf))).first;
        }
        return it->second.first;
    }

    // Device view of a learned model for the learned_* kernels.
    LearnedProjection learned_projection() {
        const DeviceProjection dp = device_buffers();
        LearnedProjection lp;
        lp.p = dp.p;
        lp.z = dp.z;
        lp.p4 = dp.p4;
        lp.z4 = dp.z4;
        lp.diag = dp.diag;
        lp.d = (uint32_t)d;
        lp.d_pad = (uint32_t)d_pad;
        lp.rht_inv = 1.0f / std::sqrt((float)d_pad);  // (n as f32).sqrt().recip(), incoherence.rs:66
        return lp;
    }

    static size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }
};

// ---------------------------------------------------------------------------
// .slhw projection files (scirust/src/weights.rs:8-31): little-endian
//   v1: magic "SLHW" u32, version u32 = 1, d u32, seed u64, rht u8, 3 zero bytes,
//       f32 P[128][d]
//   v2: the same 24-byte header, then u32 FNV-1a of (header, payload), then P.
// Checks and messages follow weights.rs:159-270 (from_bytes) and :292-311 (load).

constexpr uint32_t kSlhwMagic = 0x534C4857u;        // "SLHW"
constexpr size_t kSlhwCommonHeader = 24;
constexpr size_t kSlhwHeaderV2 = 28;
constexpr uint64_t kSlhwMaxBytes = 256ull << 20;   // weights.rs:289

uint32_t fnv1a(const uint8_t* a, size_t na, const uint8_t* b, size_t nb) {  // weights.rs:68-81
    uint32_t h = 0x811C9DC5u;
    for (size_t i = 0; i < na; ++i) h = (h ^ a[i]) * 0x01000193u;
    for (size_t i = 0; i < nb; ++i) h = (h ^ b[i]) * 0x01000193u;
    return h;
}

uint32_t le32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

size_t next_pow2(size_t n) {  // incoherence.rs:29-35
    size_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

std::shared_ptr<Model> parse_slhw(const std::vector<uint8_t>& bytes) {
    const size_t n = bytes.size();
    if (n < kSlhwCommonHeader) fail(SLHA_ERR_IO, "weights: truncated header");
    const uint8_t* b = bytes.data();
    if (le32(b) != kSlhwMagic) fail(SLHA_ERR_IO, "weights: bad magic (not an SLHW file)");
    const uint32_t version = le32(b + 4);
    if (version != 1 && version != 2)
        fail(SLHA_ERR_IO, "weights: unsupported version %u (supported: 1 and 2)", version);
    const size_t header = version == 1 ? kSlhwCommonHeader : kSlhwHeaderV2;
    if (n < header) fail(SLHA_ERR_IO, "weights: truncated header");
    const uint32_t d = le32(b + 8);
    if (d <= 128) fail(SLHA_ERR_IO, "weights: invalid dimension %u (must be greater than D_C=128)", d);
    uint64_t seed = 0;
    for (int i = 7; i >= 0; --i) seed = (seed << 8) | b[12 + i];
    if (b[20] > 1) fail(SLHA_ERR_IO, "weights: invalid RHT flag %u (expected 0 or 1)", (unsigned)b[20]);
    const bool rht = b[20] == 1;
    if (b[21] || b[22] || b[23]) fail(SLHA_ERR_IO, "weights: non-zero reserved header bytes");
    const uint64_t expected = (uint64_t)header + (uint64_t)128 * d * 4;
    if (n != expected)
        fail(SLHA_ERR_IO, "weights: size mismatch (got %zu, expected %llu)", n,
             (unsigned long long)expected);
    if (version == 2) {
        const uint32_t stored = le32(b + kSlhwCommonHeader);
        const uint32_t calc = fnv1a(b, kSlhwCommonHeader, b + header, n - header);
        if (stored != calc)
            fail(SLHA_ERR_IO, "weights: checksum mismatch (stored 0x%08x, calculated 0x%08x)",
                 stored, calc);
    }
    auto m = std::make_shared<Model>();
    m->learned = true;
    m->d = d;
    m->seed = seed;
    m->rht = rht;
    m->p.resize((size_t)128 * d);
    for (size_t i = 0; i < m->p.size(); ++i) {
        const uint32_t u = le32(b + header + 4 * i);
        float v;
        std::memcpy(&v, &u, 4);
        if (!std::isfinite(v))
            fail(SLHA_ERR_IO, "weights: non-finite projection value at index %zu", i);
        m->p[i] = v;
    }
    // LearnedModel::try_from_projection_with (learned.rs:218-250): d_pad,
    // RHT diagonal from seed ^ 0xA2A2..A2, then Z [256][d_pad] from seed.
    m->d_pad = rht ? next_pow2(d) : d;
    if (m->d_pad > kLearnedMaxDPad)
        fail(SLHA_ERR_IO,
             "weights: d = %u (padded %zu) exceeds this build's GPU limit of %u padded dimensions",
             d, m->d_pad, kLearnedMaxDPad);
    m->diag.assign(m->d_pad, 1.0f);
    if (rht) {
        Rng r(seed ^ 0xA2A2A2A2A2A2A2A2ull);
        for (auto& x : m->diag) x = r.next_unit() < 0.5f ? -1.0f : 1.0f;
    }
    m->z.resize((size_t)256 * m->d_pad);
    Rng r(seed);
    for (auto& x : m->z) x = r.next_gaussian();
    return m;
}

std::shared_ptr<Model> load_slhw(const char* path) {  // weights.rs:292-311
    struct stat st;
    if (::stat(path, &st) != 0)
        fail(SLHA_ERR_IO, "weights: cannot stat %s: %s", path, std::strerror(errno));
    if (!S_ISREG(st.st_mode))
        fail(SLHA_ERR_IO, "weights: %s is not a regular file (refusing to read a FIFO/device)", path);
    if ((uint64_t)st.st_size > kSlhwMaxBytes)
        fail(SLHA_ERR_IO, "weights: %s is %llu bytes, above the %llu-byte safety cap", path,
             (unsigned long long)st.st_size, (unsigned long long)kSlhwMaxBytes);
    std::FILE* f = std::fopen(path, "rb");
    if (!f) fail(SLHA_ERR_IO, "weights: cannot read %s: %s", path, std::strerror(errno));
    std::vector<uint8_t> bytes((size_t)st.st_size);
    const size_t got = bytes.empty() ? 0 : std::fread(bytes.data(), 1, bytes.size(), f);
    std::fclose(f);
    if (got != bytes.size()) fail(SLHA_ERR_IO, "weights: cannot read %s: short read", path);
    return parse_slhw(bytes);
}

}  // namespace

struct SlhaModel {
    uint64_t opaque;
};
struct SlhaContext {
    ContextObj obj;
};

namespace {

struct Registry {
    std::shared_mutex mu;
    std::unordered_map<uintptr_t, std::pair<std::unique_ptr<SlhaModel>, std::shared_ptr<Model>>> live;
    std::vector<std::unique_ptr<SlhaModel>> retired;
};

Registry& registry() {
    static Registry* r = new Registry();  // never destroyed: handles outlive static teardown
    return *r;
}

SlhaModel* register_model(std::shared_ptr<Model> m) {
    auto token = std::make_unique<SlhaModel>();
    token->opaque = 0;
    SlhaModel* p = token.get();
    auto& r = registry();
    std::unique_lock<std::shared_mutex> lock(r.mu);
    r.live.emplace(reinterpret_cast<uintptr_t>(p), std::make_pair(std::move(token), std::move(m)));
    return p;
}

std::shared_ptr<Model> model_of(const SlhaModel* model) {  // lib.rs:170-194
    if (!model) fail(SLHA_ERR_NULL, "model handle is NULL");
    if (reinterpret_cast<uintptr_t>(model) % alignof(SlhaModel) != 0)
        fail(SLHA_ERR_INVALID_HANDLE, "model handle is misaligned");
    auto& r = registry();
    std::shared_lock<std::shared_mutex> lock(r.mu);
    auto it = r.live.find(reinterpret_cast<uintptr_t>(model));
    if (it == r.live.end()) fail(SLHA_ERR_INVALID_HANDLE, "model handle is not a live SLHA handle");
    return it->second.second;
}

// ---------------------------------------------------------------------------
// Validation (lib.rs:233-286)

void validate_finite(const float* v, size_t n, const char* name) {
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(v[i])) fail(SLHA_ERR_NONFINITE, "%s[%zu] is not finite", name, i);
}

void validate_tile(const SciRustSlhaTile& t) {
    const uint16_t known = SLHA_FLAG_WARM | SLHA_FLAG_NF4 | SLHA_FLAG_MIXED | SLHA_FLAG_TQ3 |
                           SLHA_FLAG_TQ3_NOCORR | SLHA_FLAG_MIX3;
    const uint16_t codecs = SLHA_FLAG_NF4 | SLHA_FLAG_MIXED | SLHA_FLAG_TQ3 | SLHA_FLAG_MIX3;
    if (t.flags & (uint16_t)~known)
        fail(SLHA_ERR_INVALID_TILE, "tile contains unknown flag bits: 0x%04x", t.flags);
    if (__builtin_popcount(t.flags & codecs) > 1)
        fail(SLHA_ERR_INVALID_TILE, "tile selects more than one latent codec");
    if ((t.flags & SLHA_FLAG_TQ3_NOCORR) && !(t.flags & (SLHA_FLAG_TQ3 | SLHA_FLAG_MIX3)))
        fail(SLHA_ERR_INVALID_TILE, "correction-drop flag requires the TQ3 or MIX3 codec");
    if (!std::isfinite(t.scale) || !std::isfinite(t.dynamic_lambda) ||
        !std::isfinite(t.residual_sigma))
        fail(SLHA_ERR_NONFINITE, "tile metadata contains a non-finite float");
    if (t.scale < 0.0f || t.dynamic_lambda < 0.0f || t.residual_sigma < 0.0f)
        fail(SLHA_ERR_INVALID_TILE,
             "tile scale, dynamic lambda, and residual sigma must be non-negative");
}

SciRustSlhaTile read_tile(const SciRustSlhaTile* p) {  // unaligned-safe read
    SciRustSlhaTile t;
    std::memcpy(&t, p, sizeof t);
    return t;
}

// ---------------------------------------------------------------------------
// Per-thread device staging for host-pointer entry points

struct Staging {
    int device = -1;
    hipStream_t stream = nullptr;
    void* buf = nullptr;
    size_t cap = 0;
};
thread_local Staging g_staging;

void require_device() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        fail(SLHA_ERR_DEVICE, "no HIP device is available to the SLHA library");
}

// Returns a device buffer of at least `bytes` bytes and the thread's stream.
char* staging(size_t bytes, hipStream_t* stream) {
    require_device();
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    Staging& s = g_staging;
    if (s.device != device) {
        s.device = device;
        s.stream = nullptr;
        s.buf = nullptr;
        s.cap = 0;
        check_hip(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking), "hipStreamCreate");
    }
    if (s.cap < bytes) {
        if (s.buf) check_hip(hipFree(s.buf), "hipFree(staging)");
        s.buf = nullptr;
        s.cap = 0;
        const size_t cap = bytes < (1u << 20) ? (1u << 20) : bytes;
        check_hip(hipMalloc(&s.buf, cap), "hipMalloc(staging)");
        s.cap = cap;
    }
    *stream = s.stream;
    return static_cast<char*>(s.buf);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Device workspace of the stream-ordered entry points (the paged top-k's
// candidate lists), one grow-only buffer per (device, stream): work queued on
// one stream never shares it with work on another. Buffers live until the
// process ends.
struct WorkspaceKey {
    int device;
    hipStream_t stream;
    bool operator==(const WorkspaceKey& o) const { return device == o.device && stream == o.stream; }
};
struct WorkspaceKeyHash {
    size_t operator()(const WorkspaceKey& k) const {
        return std::hash<void*>()(static_cast<void*>(k.stream)) ^ (size_t)k.device * 0x9E3779B97F4A7C15ull;
    }
};
struct Workspace {
    void* buf = nullptr;
    size_t cap = 0;
};
std::mutex g_workspace_mu;
std::unordered_map<WorkspaceKey, Workspace, WorkspaceKeyHash> g_workspaces;

void* stream_workspace(size_t bytes, hipStream_t stream) {
    if (bytes == 0) return nullptr;
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_workspace_mu);
    Workspace& w = g_workspaces[WorkspaceKey{device, stream}];
    if (w.cap < bytes) {
        if (w.buf) {
            // the old buffer may still be read by work queued on this stream
            check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
            check_hip(hipFree(w.buf), "hipFree(workspace)");
        }
        w.buf = nullptr;
        w.cap = 0;
        check_hip(hipMalloc(&w.buf, bytes), "hipMalloc(workspace)");
        w.cap = bytes;
    }
    return w.buf;
}

// GPU eq. 2.3 (exact order) over host tiles; scores written to host `out`.
void score_host_tiles(const SciRustSlhaTile* tiles, size_t n, const float* qc, const uint64_t* qs,
                      float* out) {
    const size_t tb = align256(n * sizeof(SciRustSlhaTile));
    const size_t qb = align256(128 * sizeof(float) + 4 * sizeof(uint64_t));
    hipStream_t s;
    char* base = staging(tb + qb + align256(n * sizeof(float)), &s);
    char* td = base;
    float* qcd = reinterpret_cast<float*>(base + tb);
    uint64_t* qsd = reinterpret_cast<uint64_t*>(base + tb + 128 * sizeof(float));
    float* sd = reinterpret_cast<float*>(base + tb + qb);
    check_hip(hipMemcpyAsync(td, tiles, n * sizeof(SciRustSlhaTile), hipMemcpyHostToDevice, s), "H2D tiles");
    check_hip(hipMemcpyAsync(qcd, qc, 128 * sizeof(float), hipMemcpyHostToDevice, s), "H2D q_coarse");
    check_hip(hipMemcpyAsync(qsd, qs, 4 * sizeof(uint64_t), hipMemcpyHostToDevice, s), "H2D q_sign");
    check_hip(launch_score_rows(td, 1, (uint32_t)n, 1, qcd, qsd, true, sd, nullptr, nullptr, -1, s),
              "score kernel");
    check_hip(hipMemcpyAsync(out, sd, n * sizeof(float), hipMemcpyDeviceToHost, s), "D2H scores");
    check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
}

std::string json_escape(const char* s) {
    std::string o;
    for (; *s; ++s) {
        if (*s == '"' || *s == '\\') o.push_back('\\');
        if ((unsigned char)*s >= 0x20) o.push_back(*s);
    }
    return o;
}

}  // namespace

// ===========================================================================
// slha.h

extern "C" {

uint32_t slha_abi_version(void) { return SLHA_ABI_VERSION; }
size_t slha_tile_size(void) { return sizeof(SciRustSlhaTile); }
size_t slha_tile_align(void) { return alignof(SciRustSlhaTile); }

const char* slha_last_error_message(void) { return g_last_error; }
void slha_clear_error(void) { clear_error(); }

SlhaContext* slha_init(void) {
    clear_error();
    return reinterpret_cast<SlhaContext*>(&g_context);
}

int32_t slha_shutdown(SlhaContext* context) {
    clear_error();
    if (!context) return SLHA_OK;
    if (context != reinterpret_cast<SlhaContext*>(&g_context)) {
        set_error("context handle was not returned by slha_init");
        return SLHA_ERR_INVALID_HANDLE;
    }
    return SLHA_OK;
}

int32_t slha_process_tile(const SciRustSlhaTile* tile, const float* q_coarse,
                          const uint64_t* q_sign, float* score_out) {
    return ffi_status([&] {
        if (!tile || !q_coarse || !q_sign || !score_out)
            fail(SLHA_ERR_NULL, "slha_process_tile received a NULL pointer");
        const SciRustSlhaTile t = read_tile(tile);
        float qc[128];
        uint64_t qs[4];
        std::memcpy(qc, q_coarse, sizeof qc);
        std::memcpy(qs, q_sign, sizeof qs);
        validate_tile(t);
        validate_finite(qc, 128, "q_coarse");
        float score = 0.0f;
        score_host_tiles(&t, 1, qc, qs, &score);
        if (!std::isfinite(score))
            fail(SLHA_ERR_NONFINITE, "tile scoring produced a non-finite result");
        std::memcpy(score_out, &score, sizeof score);
    });
}

int32_t slha_prepare_query(const SlhaModel* model, const float* q, size_t d, float* q_coarse,
                           uint64_t* q_sign) {
    return ffi_status([&] {
        if (!q || !q_coarse || !q_sign)
            fail(SLHA_ERR_NULL, "slha_prepare_query received a NULL data pointer");
        auto m = model_of(model);
        if (d != m->d)
            fail(SLHA_ERR_DIMENSION, "query dimension mismatch: received %zu, expected %zu", d, m->d);
        std::vector<float> qv(d);
        std::memcpy(qv.data(), q, d * sizeof(float));
        validate_finite(qv.data(), d, "q");
        hipStream_t s;
        const size_t qb = align256(d * sizeof(float));
        char* base = staging(qb + align256(512) + align256(32), &s);
        float* qd = reinterpret_cast<float*>(base);
        float* qcd = reinterpret_cast<float*>(base + qb);
        uint64_t* qsd = reinterpret_cast<uint64_t*>(base + qb + 512);
        check_hip(hipMemcpyAsync(qd, qv.data(), d * sizeof(float), hipMemcpyHostToDevice, s), "H2D q");
        if (m->learned) {
            check_hip(launch_learned_prepare(qd, kDtypeF32, 1, m->learned_projection(), qcd, qsd, s),
                      "learned prepare kernel");
        } else {
            auto zb = m->device_buffers();
            check_hip(launch_prepare_queries(qd, kDtypeF32, 1, zb.z, zb.diag, rht_inv(), qcd, qsd, s),
                      "prepare kernel");
        }
        float qc[128];
        uint64_t qs[4];
        check_hip(hipMemcpyAsync(qc, qcd, sizeof qc, hipMemcpyDeviceToHost, s), "D2H q_coarse");
        check_hip(hipMemcpyAsync(qs, qsd, sizeof qs, hipMemcpyDeviceToHost, s), "D2H q_sign");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        validate_finite(qc, 128, "q_coarse");
        std::memcpy(q_coarse, qc, sizeof qc);
        std::memcpy(q_sign, qs, sizeof qs);
    });
}

int32_t slha_score_tile(const SlhaModel* model, const SciRustSlhaTile* tile, const float* q_coarse,
                        const uint64_t* q_sign, float* score_out) {
    return ffi_status([&] {
        if (!tile || !q_coarse || !q_sign || !score_out)
            fail(SLHA_ERR_NULL, "slha_score_tile received a NULL pointer");
        (void)model_of(model);
        const SciRustSlhaTile t = read_tile(tile);
        float qc[128];
        uint64_t qs[4];
        std::memcpy(qc, q_coarse, sizeof qc);
        std::memcpy(qs, q_sign, sizeof qs);
        validate_tile(t);
        validate_finite(qc, 128, "q_coarse");
        float score = 0.0f;
        score_host_tiles(&t, 1, qc, qs, &score);
        if (!std::isfinite(score))
            fail(SLHA_ERR_NONFINITE, "tile scoring produced a non-finite result");
        std::memcpy(score_out, &score, sizeof score);
    });
}

int32_t slha_score_tiles(const SlhaModel* model, const SciRustSlhaTile* tiles, size_t n_tiles,
                         const float* q_coarse, const uint64_t* q_sign, float* scores_out) {
    return ffi_status([&] {
        if (!tiles || !q_coarse || !q_sign || !scores_out)
            fail(SLHA_ERR_NULL, "slha_score_tiles received a NULL pointer");
        (void)model_of(model);
        const size_t kMaxTiles = size_t(1) << 20;  // lib.rs:207-208
        if (n_tiles > kMaxTiles)
            fail(SLHA_ERR_DIMENSION, "n_tiles=%zu exceeds the safety bound %zu", n_tiles, kMaxTiles);
        if (n_tiles == 0) return;
        float qc[128];
        uint64_t qs[4];
        std::memcpy(qc, q_coarse, sizeof qc);
        std::memcpy(qs, q_sign, sizeof qs);
        validate_finite(qc, 128, "q_coarse");
        std::vector<SciRustSlhaTile> tv(n_tiles);
        std::memcpy(tv.data(), tiles, n_tiles * sizeof(SciRustSlhaTile));
        for (size_t i = 0; i < n_tiles; ++i) validate_tile(tv[i]);
        std::vector<float> sv(n_tiles);
        score_host_tiles(tv.data(), n_tiles, qc, qs, sv.data());
        for (size_t i = 0; i < n_tiles; ++i)
            if (!std::isfinite(sv[i]))
                fail(SLHA_ERR_NONFINITE, "tile %zu scoring produced a non-finite result", i);
        std::memcpy(scores_out, sv.data(), n_tiles * sizeof(float));
    });
}

char* slha_audit(void) {
    clear_error();
    try {
        std::string j = "{\"abi_version\":" + std::to_string(SLHA_ABI_VERSION) +
                        ",\"tile_size\":" + std::to_string(sizeof(SciRustSlhaTile)) +
                        ",\"tile_align\":" + std::to_string(alignof(SciRustSlhaTile)) +
                        ",\"layout_ok\":true";
        int n = 0;
        if (hipGetDeviceCount(&n) == hipSuccess && n > 0) {
            int dev = 0;
            hipDeviceProp_t prop;
            if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
                j += ",\"device\":\"" + json_escape(prop.name) + "\",\"arch\":\"" +
                     json_escape(prop.gcnArchName) + "\"";
            // Known answer (scirust/examples/basic_usage.rs:9-45): a ramp
            // (i-64)/16 quantised with codec INT4_SINGLE, lambda 0.5,
            // q0 = q1 = 1, q_sign = 0x123456789ABCDEF0 x4 scores exactly -8.
            std::shared_ptr<Model> m = std::make_shared<Model>();
            m->z.assign(256 * 128, 0.0f);
            m->diag.assign(128, 1.0f);
            float key[128];
            for (int i = 0; i < 128; ++i) key[i] = ((float)i - 64.0f) / 16.0f;
            hipStream_t s;
            char* base = staging(4096, &s);
            check_hip(hipMemcpyAsync(base, key, sizeof key, hipMemcpyHostToDevice, s), "H2D key");
            auto zb = m->device_buffers();
            check_hip(launch_encode(base, kDtypeF32, 1, 1, 1, 0, kCodecInt4Single, kResidualZ, 0,
                                    zb.z, nullptr, 0.0f, nullptr, lambda_c(), rht_inv(), base + 1024,
                                    s),
                      "encode kernel");
            SciRustSlhaTile t;
            check_hip(hipMemcpyAsync(&t, base + 1024, sizeof t, hipMemcpyDeviceToHost, s), "D2H tile");
            check_hip(hipStreamSynchronize(s), "sync");
            t.dynamic_lambda = 0.5f;
            float qc[128] = {0};
            qc[0] = qc[1] = 1.0f;
            uint64_t qs[4] = {0x123456789ABCDEF0ull, 0x123456789ABCDEF0ull, 0x123456789ABCDEF0ull,
                              0x123456789ABCDEF0ull};
            float score = 0.0f;
            score_host_tiles(&t, 1, qc, qs, &score);
            char buf[64];
            std::snprintf(buf, sizeof buf, "%.6f", (double)score);
            j += std::string(",\"kat_basic_usage\":") + buf + ",\"ok\":" + (score == -8.0f ? "true" : "false");
        } else {
            j += ",\"device\":null,\"ok\":false";
        }
        j += "}";
        char* out = static_cast<char*>(std::malloc(j.size() + 1));
        if (!out) return nullptr;
        std::memcpy(out, j.c_str(), j.size() + 1);
        return out;
    } catch (const SlhaError& e) {
        set_error(e.msg);
        return nullptr;
    } catch (...) {
        set_error("panic caught while running the SLHA self-audit");
        return nullptr;
    }
}

void slha_free_string(char* string) { std::free(string); }

SlhaModel* slha_weights_load(const char* path) {
    clear_error();
    if (!path) {
        set_error("weights path is NULL");
        return nullptr;
    }
    // Reject invalid UTF-8 like CStr::to_str (lib.rs:658-661).
    const unsigned char* p = reinterpret_cast<const unsigned char*>(path);
    while (*p) {
        int extra = (*p < 0x80) ? 0 : ((*p >> 5) == 0x6) ? 1 : ((*p >> 4) == 0xE) ? 2 : ((*p >> 3) == 0x1E) ? 3 : -1;
        if (extra < 0) {
            set_error("weights path is not valid UTF-8");
            return nullptr;
        }
        ++p;
        for (int i = 0; i < extra; ++i, ++p)
            if ((*p & 0xC0) != 0x80) {
                set_error("weights path is not valid UTF-8");
                return nullptr;
            }
    }
    SlhaModel* out = nullptr;
    const int32_t rc = ffi_status([&] { out = register_model(load_slhw(path)); });
    return rc == SLHA_OK ? out : nullptr;
}

size_t slha_model_dim(const SlhaModel* model) {
    size_t d = 0;
    const int32_t rc = ffi_status([&] { d = model_of(model)->d; });
    return rc == SLHA_OK ? d : 0;
}

int32_t slha_encode_key(const SlhaModel* model, const float* key, size_t d, uint32_t position,
                        int32_t codec, SciRustSlhaTile* out_tile) {
    return ffi_status([&] {
        if (!key || !out_tile) fail(SLHA_ERR_NULL, "slha_encode_key received a NULL data pointer");
        auto m = model_of(model);
        if (d != m->d)
            fail(SLHA_ERR_DIMENSION, "key dimension mismatch: received %zu, expected %zu", d, m->d);
        if (codec < 0 || codec > 5)
            fail(SLHA_ERR_CODEC, "unknown codec id %d; expected an integer from 0 to 5", codec);
        std::vector<float> kv(d);
        std::memcpy(kv.data(), key, d * sizeof(float));
        validate_finite(kv.data(), d, "key");
        hipStream_t s;
        const size_t kb = align256(d * sizeof(float));
        char* base = staging(kb + 256, &s);
        check_hip(hipMemcpyAsync(base, kv.data(), d * sizeof(float), hipMemcpyHostToDevice, s),
                  "H2D key");
        if (m->learned) {  // LearnedModel::encode_with (learned.rs:353-408)
            check_hip(launch_learned_encode(base, kDtypeF32, 1, 1, 1, position, codec, 0,
                                            m->learned_projection(), lambda_c(), base + kb, s),
                      "learned encode kernel");
        } else {
            auto zb = m->device_buffers();
            check_hip(launch_encode(base, kDtypeF32, 1, 1, 1, position, codec, m->residual_mode, 0,
                                    zb.z, zb.zpack, zb.cert_scale, zb.diag, lambda_c(), rht_inv(),
                                    base + kb, s),
                      "encode kernel");
        }
        SciRustSlhaTile t;
        check_hip(hipMemcpyAsync(&t, base + kb, sizeof t, hipMemcpyDeviceToHost, s), "D2H tile");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        validate_tile(t);
        std::memcpy(out_tile, &t, sizeof t);
    });
}

static int32_t decode_common(const SlhaModel* model, const SciRustSlhaTile* tile, float* out,
                             size_t d, bool with_residual, const char* fn) {
    return ffi_status([&] {
        if (!tile || !out) fail(SLHA_ERR_NULL, "%s received a NULL data pointer", fn);
        auto m = model_of(model);
        if (d != m->d)
            fail(SLHA_ERR_DIMENSION, "output dimension mismatch: received %zu, expected %zu", d, m->d);
        const SciRustSlhaTile t = read_tile(tile);
        validate_tile(t);
        hipStream_t s;
        char* base = staging(256 + align256(d * sizeof(float)), &s);
        float* od = reinterpret_cast<float*>(base + 256);
        check_hip(hipMemcpyAsync(base, &t, sizeof t, hipMemcpyHostToDevice, s), "H2D tile");
        if (m->learned) {  // reconstruct / reconstruct_from_tile (learned.rs:276-320)
            check_hip(launch_learned_decode(base, 1, m->learned_projection(), with_residual ? 1 : 0,
                                            sqrt_half_pi(), od, s),
                      "learned decode kernel");
        } else {
            auto zb = m->device_buffers();
            const float* z = (with_residual && !m->rht) ? zb.z : nullptr;
            check_hip(launch_decode(base, 1, z, sqrt_half_pi(), od, s), "decode kernel");
        }
        std::vector<float> v(d);
        check_hip(hipMemcpyAsync(v.data(), od, d * sizeof(float), hipMemcpyDeviceToHost, s), "D2H");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        validate_finite(v.data(), d, with_residual || m->learned ? "reconstruction" : "dequantized_latent");
        std::memcpy(out, v.data(), d * sizeof(float));
    });
}

int32_t slha_decode_latent(const SlhaModel* model, const SciRustSlhaTile* tile, float* out,
                           size_t d) {
    return decode_common(model, tile, out, d, false, "slha_decode_latent");
}

int32_t slha_decode_key(const SlhaModel* model, const SciRustSlhaTile* tile, float* out, size_t d) {
    return decode_common(model, tile, out, d, true, "slha_decode_key");
}

int32_t slha_weights_release(SlhaModel* model) {
    if (!model) {
        clear_error();
        return SLHA_OK;
    }
    return ffi_status([&] {
        if (reinterpret_cast<uintptr_t>(model) % alignof(SlhaModel) != 0)
            fail(SLHA_ERR_INVALID_HANDLE, "model handle is misaligned");
        auto& r = registry();
        std::shared_ptr<Model> victim;
        {
            std::unique_lock<std::shared_mutex> lock(r.mu);
            auto it = r.live.find(reinterpret_cast<uintptr_t>(model));
            if (it == r.live.end())
                fail(SLHA_ERR_INVALID_HANDLE, "model handle is not a live SLHA handle");
            r.retired.push_back(std::move(it->second.first));
            victim = std::move(it->second.second);
            r.live.erase(it);
        }
    });
}

void slha_weights_free(SlhaModel* model) { (void)slha_weights_release(model); }

// ===========================================================================
// slha_gpu.h

SlhaModel* slha_model_new_raw128(uint64_t seed, int32_t rht, int32_t residual_mode) {
    SlhaModel* out = nullptr;
    const int32_t rc = ffi_status([&] {
        if (residual_mode != SLHA_RESIDUAL_Z && residual_mode != SLHA_RESIDUAL_R)
            fail(SLHA_ERR_CODEC, "unknown residual mode %d", residual_mode);
        auto m = std::make_shared<Model>();
        m->seed = seed;
        m->rht = rht != 0;
        m->residual_mode = residual_mode;
        m->diag.assign(128, 1.0f);
        if (m->rht) {  // learned.rs:158-165, incoherence.rs:89-98
            Rng r(seed ^ 0xA2A2A2A2A2A2A2A2ull);
            for (auto& x : m->diag) x = r.next_unit() < 0.5f ? -1.0f : 1.0f;
        }
        m->z.resize(256 * 128);  // scenario.rs:59-64
        Rng r(seed);
        for (auto& x : m->z) x = r.next_gaussian();
        out = register_model(std::move(m));
    });
    return rc == SLHA_OK ? out : nullptr;
}

int32_t slha_model_projection(const SlhaModel* model, float* z_out, float* rht_diag_out) {
    return ffi_status([&] {
        if (!z_out) fail(SLHA_ERR_NULL, "z_out is NULL");
        auto m = model_of(model);
        std::memcpy(z_out, m->z.data(), m->z.size() * sizeof(float));
        if (rht_diag_out) std::memcpy(rht_diag_out, m->diag.data(), m->diag.size() * sizeof(float));
    });
}

size_t slha_model_pad_dim(const SlhaModel* model) {
    size_t d_pad = 0;
    const int32_t rc = ffi_status([&] { d_pad = model_of(model)->d_pad; });
    return rc == SLHA_OK ? d_pad : 0;
}

int32_t slha_model_latent_projection(const SlhaModel* model, float* p_out) {
    return ffi_status([&] {
        if (!p_out) fail(SLHA_ERR_NULL, "p_out is NULL");
        auto m = model_of(model);
        if (!m->learned) {  // identity latent
            std::memset(p_out, 0, 128 * 128 * sizeof(float));
            for (int k = 0; k < 128; ++k) p_out[k * 128 + k] = 1.0f;
            return;
        }
        std::memcpy(p_out, m->p.data(), m->p.size() * sizeof(float));
    });
}

int32_t slha_gpu_encode(const SlhaModel* model, const void* keys_dev, int32_t key_dtype,
                        size_t n_rows, size_t n_tok, size_t n_kv_heads, uint32_t pos0,
                        int32_t codec, int32_t warm, SciRustSlhaTile* tiles_dev, void* stream) {
    return ffi_status([&] {
        auto m = model_of(model);
        if (codec < 0 || codec > 5)
            fail(SLHA_ERR_CODEC, "unknown codec id %d; expected an integer from 0 to 5", codec);
        if (key_dtype != SLHA_DTYPE_F32 && key_dtype != SLHA_DTYPE_BF16)
            fail(SLHA_ERR_DIMENSION, "unknown key dtype %d", key_dtype);
        if (n_kv_heads == 0 || n_kv_heads > 65536)
            fail(SLHA_ERR_DIMENSION, "n_kv_heads=%zu out of range", n_kv_heads);
        if (n_tok > 0xFFFFFFFFull || n_rows * n_tok >= (1ull << 40))
            fail(SLHA_ERR_DIMENSION, "batch too large: %zu rows x %zu tokens", n_rows, n_tok);
        const uint64_t n = (uint64_t)n_rows * n_tok;
        if (n == 0) return;
        if (!keys_dev || !tiles_dev) fail(SLHA_ERR_NULL, "slha_gpu_encode received a NULL pointer");
        require_device();
        if (m->learned) {
            check_hip(launch_learned_encode(keys_dev, key_dtype, n, (uint32_t)n_tok,
                                            (uint32_t)n_kv_heads, pos0, codec, warm,
                                            m->learned_projection(), lambda_c(), tiles_dev,
                                            static_cast<hipStream_t>(stream)),
                      "learned encode kernel");
            return;
        }
        auto zb = m->device_buffers();
        check_hip(launch_encode(keys_dev, key_dtype, n, (uint32_t)n_tok, (uint32_t)n_kv_heads, pos0,
                                codec, m->residual_mode, warm, zb.z, zb.zpack, zb.cert_scale,
                                zb.diag, lambda_c(), rht_inv(), tiles_dev,
                                static_cast<hipStream_t>(stream)),
                  "encode kernel");
    });
}

int32_t slha_gpu_prepare_queries(const SlhaModel* model, const void* q_dev, int32_t q_dtype,
                                 size_t n_q, float* q_coarse_dev, uint64_t* q_sign_dev,
                                 void* stream) {
    return ffi_status([&] {
        auto m = model_of(model);
        if (q_dtype != SLHA_DTYPE_F32 && q_dtype != SLHA_DTYPE_BF16)
            fail(SLHA_ERR_DIMENSION, "unknown query dtype %d", q_dtype);
        if (n_q == 0) return;
        if (!q_dev || !q_coarse_dev || !q_sign_dev)
            fail(SLHA_ERR_NULL, "slha_gpu_prepare_queries received a NULL pointer");
        require_device();
        if (m->learned) {
            check_hip(launch_learned_prepare(q_dev, q_dtype, n_q, m->learned_projection(),
                                             q_coarse_dev, q_sign_dev,
                                             static_cast<hipStream_t>(stream)),
                      "learned prepare kernel");
            return;
        }
        auto zb = m->device_buffers();
        check_hip(launch_prepare_queries(q_dev, q_dtype, n_q, zb.z, zb.diag, rht_inv(),
                                         q_coarse_dev, q_sign_dev, static_cast<hipStream_t>(stream)),
                  "prepare kernel");
    });
}

int32_t slha_gpu_score(const SciRustSlhaTile* tiles_dev, size_t n_rows, size_t n_tok,
                       const float* q_coarse_dev, const uint64_t* q_sign_dev, size_t group,
                       int32_t mode, float* scores_dev, uint32_t* hamming_dev, void* stream) {
    return slha_gpu_score_codec(tiles_dev, n_rows, n_tok, q_coarse_dev, q_sign_dev, group, mode,
                                -1, scores_dev, hamming_dev, stream);
}

int32_t slha_gpu_score_codec(const SciRustSlhaTile* tiles_dev, size_t n_rows, size_t n_tok,
                             const float* q_coarse_dev, const uint64_t* q_sign_dev, size_t group,
                             int32_t mode, int32_t codec_hint, float* scores_dev,
                             uint32_t* hamming_dev, void* stream) {
    return ffi_status([&] {
        if (mode != SLHA_SCORE_FAST && mode != SLHA_SCORE_EXACT)
            fail(SLHA_ERR_DIMENSION, "unknown score mode %d", mode);
        if (codec_hint < -1 || codec_hint > SLHA_CODEC_MIX3)
            fail(SLHA_ERR_CODEC, "unknown codec hint %d", codec_hint);
        if (group == 0 || group > kMaxGroup)
            fail(SLHA_ERR_DIMENSION, "group=%zu must be in [1, %u]", group, kMaxGroup);
        if (n_rows > 65535 || n_tok > 0xFFFFFFFFull)
            fail(SLHA_ERR_DIMENSION, "n_rows=%zu / n_tok=%zu out of range", n_rows, n_tok);
        if (n_rows == 0 || n_tok == 0) return;
        if (!tiles_dev || !q_coarse_dev || !q_sign_dev || !scores_dev)
            fail(SLHA_ERR_NULL, "slha_gpu_score received a NULL pointer");
        require_device();
        const hipStream_t hs = static_cast<hipStream_t>(stream);
        void* ws = stream_workspace(score_rows_workspace_bytes((uint32_t)n_rows, (uint32_t)group,
                                                               mode == SLHA_SCORE_EXACT,
                                                               hamming_dev != nullptr),
                                    hs);
        check_hip(launch_score_rows(tiles_dev, (uint32_t)n_rows, (uint32_t)n_tok, (uint32_t)group,
                                    q_coarse_dev, q_sign_dev, mode == SLHA_SCORE_EXACT, scores_dev,
                                    hamming_dev, ws, codec_hint, hs),
                  "score kernel");
    });
}

int32_t slha_gpu_validate_tiles(const SciRustSlhaTile* tiles_dev, size_t n, uint64_t* status_dev,
                                void* stream) {
    return ffi_status([&] {
        if (!status_dev) fail(SLHA_ERR_NULL, "status_dev is NULL");
        if (n > 0 && !tiles_dev) fail(SLHA_ERR_NULL, "tiles_dev is NULL");
        require_device();
        hipStream_t s = static_cast<hipStream_t>(stream);
        check_hip(launch_fill_u64(status_dev, 1, ~0ull, s), "fill kernel");
        check_hip(launch_validate(tiles_dev, n, status_dev, s), "validate kernel");
    });
}

int32_t slha_gpu_decode(const SlhaModel* model, const SciRustSlhaTile* tiles_dev, size_t n,
                        int32_t with_residual, float* out_dev, void* stream) {
    return ffi_status([&] {
        auto m = model_of(model);
        if (n == 0) return;
        if (!tiles_dev || !out_dev) fail(SLHA_ERR_NULL, "slha_gpu_decode received a NULL pointer");
        require_device();
        if (m->learned) {
            check_hip(launch_learned_decode(tiles_dev, n, m->learned_projection(),
                                            with_residual ? 1 : 0, sqrt_half_pi(), out_dev,
                                            static_cast<hipStream_t>(stream)),
                      "learned decode kernel");
            return;
        }
        auto zb = m->device_buffers();
        const float* z = (with_residual && !m->rht) ? zb.z : nullptr;
        check_hip(launch_decode(tiles_dev, n, z, sqrt_half_pi(), out_dev,
                                static_cast<hipStream_t>(stream)),
                  "decode kernel");
    });
}

}  // extern "C"

namespace {

// Argument checks shared by the two paged entry points; returns log2(page_tiles),
// or -1 when there is no work (n_seq == 0 or max_len == 0).
int paged_checks(const SciRustSlhaTile* arena_dev, size_t page_tiles, const uint32_t* page_table_dev,
                 size_t max_pages, const uint32_t* seq_len_dev, const uint64_t* score_base_dev,
                 size_t n_seq, size_t max_len, size_t n_kv_heads, size_t group,
                 const float* q_coarse_dev, const uint64_t* q_sign_dev, float* scores_dev, size_t k,
                 uint32_t* topk_idx_dev, float* topk_score_dev, const char* fn) {
    if (page_tiles == 0 || (page_tiles & (page_tiles - 1)) != 0 || page_tiles > (1u << 30))
        fail(SLHA_ERR_DIMENSION, "page_tiles=%zu must be a power of two", page_tiles);
    if (group == 0 || group > kMaxGroup)
        fail(SLHA_ERR_DIMENSION, "group=%zu must be in [1, %u]", group, kMaxGroup);
    if (k > kMaxTopK) fail(SLHA_ERR_DIMENSION, "k=%zu exceeds %u", k, kMaxTopK);
    if (k > 0 && (max_len + kTopkSeg - 1) / kTopkSeg * k > kTopkMaxCandidates)
        fail(SLHA_ERR_DIMENSION,
             "top-k of rows up to max_len=%zu needs ceil(max_len/%u)*k <= %u (k=%zu)",
             max_len, kTopkSeg, kTopkMaxCandidates, k);
    if (n_kv_heads == 0 || n_seq * n_kv_heads > 65535 || max_len > 0xFFFFFFFFull ||
        max_pages > 0xFFFFFFFFull || (uint64_t)max_len > (uint64_t)max_pages * page_tiles)
        fail(SLHA_ERR_DIMENSION, "paged geometry out of range (n_seq=%zu n_kv=%zu max_len=%zu)",
             n_seq, n_kv_heads, max_len);
    if (n_seq == 0 || max_len == 0) return -1;
    if (!arena_dev || !page_table_dev || !seq_len_dev || !score_base_dev || !q_coarse_dev ||
        !q_sign_dev || !scores_dev || (k > 0 && (!topk_idx_dev || !topk_score_dev)))
        fail(SLHA_ERR_NULL, "%s received a NULL pointer", fn);
    require_device();
    int shift = 0;
    while ((size_t(1) << shift) < page_tiles) ++shift;
    return shift;
}

}  // namespace

extern "C" {

int32_t slha_gpu_score_paged_topk(const SciRustSlhaTile* arena_dev, size_t page_tiles,
                                  const uint32_t* page_table_dev, size_t max_pages,
                                  const uint32_t* seq_len_dev, const uint64_t* score_base_dev,
                                  size_t n_seq, size_t max_len, size_t n_kv_heads, size_t group,
                                  const float* q_coarse_dev, const uint64_t* q_sign_dev,
                                  float* scores_dev, size_t k, uint32_t* topk_idx_dev,
                                  float* topk_score_dev, void* stream) {
    return ffi_status([&] {
        const int shift = paged_checks(arena_dev, page_tiles, page_table_dev, max_pages, seq_len_dev,
                                       score_base_dev, n_seq, max_len, n_kv_heads, group, q_coarse_dev,
                                       q_sign_dev, scores_dev, k, topk_idx_dev, topk_score_dev,
                                       "slha_gpu_score_paged_topk");
        if (shift < 0) return;
        hipStream_t s = static_cast<hipStream_t>(stream);
        void* ws = k == 0 ? nullptr
                          : stream_workspace(paged_topk_workspace_bytes(
                                                 (uint32_t)n_seq, (uint32_t)max_len,
                                                 (uint32_t)n_kv_heads, (uint32_t)group, (uint32_t)k),
                                             s);
        check_hip(launch_score_paged_topk(arena_dev, (uint32_t)shift, page_table_dev, (uint32_t)max_pages,
                                          seq_len_dev, score_base_dev, (uint32_t)n_seq,
                                          (uint32_t)max_len, (uint32_t)n_kv_heads, (uint32_t)group,
                                          q_coarse_dev, q_sign_dev, scores_dev, (uint32_t)k,
                                          topk_idx_dev, topk_score_dev, ws, s),
                  "paged score kernel");
    });
}

static_assert(SLHA_NOALLOC_SCRATCH_BYTES == kNoAllocScratchBytes, "header and library agree on the scratch size");

int32_t slha_gpu_score_paged_topk_noalloc(const SciRustSlhaTile* arena_dev, size_t page_tiles,
                                          const uint32_t* page_table_dev, size_t max_pages,
                                          const uint32_t* seq_len_dev, const uint64_t* score_base_dev,
                                          size_t n_seq, size_t max_len, size_t n_kv_heads, size_t group,
                                          const float* q_coarse_dev, const uint64_t* q_sign_dev,
                                          float* scores_dev, size_t k, uint32_t* topk_idx_dev,
                                          float* topk_score_dev, void* stream) {
    return ffi_status([&] {
        const int shift = paged_checks(arena_dev, page_tiles, page_table_dev, max_pages, seq_len_dev,
                                       score_base_dev, n_seq, max_len, n_kv_heads, group, q_coarse_dev,
                                       q_sign_dev, scores_dev, k, topk_idx_dev, topk_score_dev,
                                       "slha_gpu_score_paged_topk_noalloc");
        if (shift < 0) return;
        const size_t need = k == 0 ? 0
                                   : paged_topk_workspace_bytes((uint32_t)n_seq, (uint32_t)max_len,
                                                                (uint32_t)n_kv_heads, (uint32_t)group,
                                                                (uint32_t)k);
        if (need > kNoAllocScratchBytes)
            fail(SLHA_ERR_DIMENSION,
                 "top-k candidates need %zu bytes (n_seq*n_kv*group*ceil(max_len/%u)*k*8); the "
                 "no-allocation entry point holds %zu",
                 need, kTopkSeg, kNoAllocScratchBytes);
        check_hip(launch_score_paged_topk_noalloc(arena_dev, (uint32_t)shift, page_table_dev,
                                                  (uint32_t)max_pages, seq_len_dev, score_base_dev,
                                                  (uint32_t)n_seq, (uint32_t)max_len, (uint32_t)n_kv_heads,
                                                  (uint32_t)group, q_coarse_dev, q_sign_dev, scores_dev,
                                                  (uint32_t)k, topk_idx_dev, topk_score_dev,
                                                  static_cast<hipStream_t>(stream)),
                  "paged score kernel");
    });
}

int32_t slha_gpu_ccos_apply(SciRustSlhaTile* tiles_dev, const uint32_t* slots_dev, size_t n,
                            int32_t op, void* stream) {
    return ffi_status([&] {
        if (op != 0 && op != 1) fail(SLHA_ERR_DIMENSION, "unknown CCOS op %d", op);
        if (n == 0) return;
        if (!tiles_dev || !slots_dev) fail(SLHA_ERR_NULL, "slha_gpu_ccos_apply received a NULL pointer");
        require_device();
        check_hip(launch_ccos_apply(tiles_dev, nullptr, slots_dev, 0, n, op, static_cast<hipStream_t>(stream)),
                  "ccos kernel");
    });
}

int32_t slha_gpu_decode_attention(const SciRustSlhaTile* tiles_dev, const void* v_dev,
                                  int32_t v_dtype, size_t n_rows, size_t n_tok, size_t d_v,
                                  const float* q_coarse_dev, const uint64_t* q_sign_dev,
                                  size_t group, float scale, float* out_dev, void* stream) {
    return ffi_status([&] {
        if (group == 0 || group > 16) fail(SLHA_ERR_DIMENSION, "group=%zu must be in [1, 16]", group);
        if (d_v != 32 && d_v != 64 && d_v != 128 && d_v != 256)
            fail(SLHA_ERR_DIMENSION, "d_v=%zu must be 32, 64, 128 or 256", d_v);
        if (v_dtype != SLHA_DTYPE_F32 && v_dtype != SLHA_DTYPE_BF16)
            fail(SLHA_ERR_DIMENSION, "unknown value dtype %d", v_dtype);
        if (n_rows > 65535 || n_tok > 0xFFFFFFFFull)
            fail(SLHA_ERR_DIMENSION, "n_rows=%zu / n_tok=%zu out of range", n_rows, n_tok);
        if (n_rows == 0) return;
        if (!out_dev) fail(SLHA_ERR_NULL, "slha_gpu_decode_attention received a NULL pointer");
        require_device();
        const hipStream_t hs = static_cast<hipStream_t>(stream);
        const uint64_t n_out = (uint64_t)n_rows * group * d_v;
        // softmax_into (metrics.rs:338): a non-finite scale, or no token at
        // all, gives all-zero weights and so a zero output.
        if (n_tok == 0 || !std::isfinite(scale)) {
            check_hip(launch_fill_u32(reinterpret_cast<uint32_t*>(out_dev), n_out, 0u, hs),
                      "fill kernel");
            return;
        }
        if (!tiles_dev || !v_dev || !q_coarse_dev || !q_sign_dev)
            fail(SLHA_ERR_NULL, "slha_gpu_decode_attention received a NULL pointer");
        void* ws = stream_workspace(decode_attention_workspace_bytes((uint32_t)n_rows, (uint32_t)n_tok,
                                                                     (uint32_t)group, (uint32_t)d_v),
                                    hs);
        check_hip(launch_decode_attention(tiles_dev, v_dev, v_dtype, (uint32_t)n_rows,
                                          (uint32_t)n_tok, (uint32_t)group, (uint32_t)d_v,
                                          q_coarse_dev, q_sign_dev, scale, out_dev, ws, hs),
                  "decode attention kernels");
    });
}

int32_t slha_gpu_synchronize(void* stream) {
    return ffi_status([&] {
        require_device();
        check_hip(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
        check_hip(hipGetLastError(), "pending HIP error");
    });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// EventLog (scirust/src/eventlog.rs): the file side on POSIX descriptors.

namespace {

constexpr uint32_t kLogMagic = SLHA_EVENTLOG_MAGIC;
constexpr uint32_t kLogV1 = 1, kLogV2 = 2;
constexpr size_t kLogHeader = SLHA_EVENTLOG_HEADER_BYTES, kLogRecord = SLHA_EVENTLOG_RECORD_BYTES;
constexpr size_t kLogChunk = 4096;  // records per read while validating

struct EventLogObj {
    int fd = -1;
    uint64_t records = 0;
    uint32_t version = kLogV2;
    bool writable = true;
    std::mutex mu;
    ~EventLogObj() {
        if (fd >= 0) ::close(fd);
    }
};

struct LogRegistry {
    std::mutex mu;
    std::unordered_map<uintptr_t, std::unique_ptr<EventLogObj>> live;
};

LogRegistry& log_registry() {
    static LogRegistry* r = new LogRegistry();
    return *r;
}

// Handles are small never-freed tokens, so a closed handle cannot alias a
// later one.
SlhaEventLog* register_log(std::unique_ptr<EventLogObj> obj) {
    SlhaEventLog* token = reinterpret_cast<SlhaEventLog*>(new uint64_t(0));
    auto& r = log_registry();
    std::lock_guard<std::mutex> lock(r.mu);
    r.live.emplace(reinterpret_cast<uintptr_t>(token), std::move(obj));
    return token;
}

EventLogObj* log_of(const SlhaEventLog* log) {
    if (!log) fail(SLHA_ERR_NULL, "EventLog handle is NULL");
    auto& r = log_registry();
    std::lock_guard<std::mutex> lock(r.mu);
    auto it = r.live.find(reinterpret_cast<uintptr_t>(log));
    if (it == r.live.end()) fail(SLHA_ERR_INVALID_HANDLE, "EventLog handle is not a live SLHA handle");
    return it->second.get();
}

[[noreturn]] void io_fail(const char* what) {
    fail(SLHA_ERR_IO, "EventLog: %s: %s", what, std::strerror(errno));
}

void write_all(int fd, const uint8_t* p, size_t n, uint64_t off) {
    while (n > 0) {
        const ssize_t w = ::pwrite(fd, p, n, (off_t)off);
        if (w < 0) {
            if (errno == EINTR) continue;
            io_fail("write");
        }
        p += w, n -= (size_t)w, off += (uint64_t)w;
    }
}

void read_all(int fd, uint8_t* p, size_t n, uint64_t off) {
    while (n > 0) {
        const ssize_t r = ::pread(fd, p, n, (off_t)off);
        if (r < 0) {
            if (errno == EINTR) continue;
            io_fail("read");
        }
        if (r == 0) fail(SLHA_ERR_IO, "EventLog: unexpected end of file");
        p += r, n -= (size_t)r, off += (uint64_t)r;
    }
}

uint64_t le64(const uint8_t* p) { return (uint64_t)le32(p) | (uint64_t)le32(p + 4) << 32; }

// eventlog.rs:148-170: FNV-1a 32 over the record's seq and slot (bytes 0..12)
// and its tile (bytes 16..144).
uint32_t record_checksum(const uint8_t* rec) {
    uint32_t h = 0x811C9DC5u;
    for (size_t i = 0; i < 12; ++i) h = (h ^ rec[i]) * 0x01000193u;
    for (size_t i = 16; i < kLogRecord; ++i) h = (h ^ rec[i]) * 0x01000193u;
    return h;
}

// decode_record (eventlog.rs:412-435): version 2 checks the stored checksum.
bool record_ok(const uint8_t* rec, uint32_t version) {
    return version != kLogV2 || le32(rec + 12) == record_checksum(rec);
}

// Visits every record in order, in chunks, failing on a bad checksum.
template <class F>
void scan_records(EventLogObj* L, F&& visit) {
    std::vector<uint8_t> buf(kLogChunk * kLogRecord);
    for (uint64_t i0 = 0; i0 < L->records; i0 += kLogChunk) {
        const size_t m = (size_t)std::min<uint64_t>(kLogChunk, L->records - i0);
        read_all(L->fd, buf.data(), m * kLogRecord, kLogHeader + i0 * kLogRecord);
        for (size_t i = 0; i < m; ++i) {
            const uint8_t* rec = buf.data() + i * kLogRecord;
            if (!record_ok(rec, L->version)) fail(SLHA_ERR_IO, "EventLog: record checksum mismatch");
            visit(i0 + i, rec);
        }
    }
}

void check_path(const char* path) {
    if (!path) fail(SLHA_ERR_NULL, "EventLog path is NULL");
}

}  // namespace

extern "C" {

SlhaEventLog* slha_eventlog_create(const char* path, int32_t exclusive) {
    SlhaEventLog* out = nullptr;
    const int32_t rc = ffi_status([&] {
        check_path(path);
        auto L = std::make_unique<EventLogObj>();
        L->fd = ::open(path, O_RDWR | O_CREAT | O_CLOEXEC | (exclusive ? O_EXCL : O_TRUNC), 0644);
        if (L->fd < 0) io_fail(exclusive && errno == EEXIST ? "refusing to overwrite an existing log" : "create");
        uint8_t h[kLogHeader] = {0};
        const uint32_t fields[3] = {kLogMagic, kLogV2, 128u};
        for (int k = 0; k < 3; ++k)
            for (int b = 0; b < 4; ++b) h[4 * k + b] = (uint8_t)(fields[k] >> (8 * b));
        write_all(L->fd, h, sizeof h, 0);
        out = register_log(std::move(L));
    });
    return rc == SLHA_OK ? out : nullptr;
}

SlhaEventLog* slha_eventlog_open(const char* path, int32_t mode) {
    SlhaEventLog* out = nullptr;
    const int32_t rc = ffi_status([&] {
        check_path(path);
        if (mode < SLHA_EVENTLOG_OPEN_STRICT || mode > SLHA_EVENTLOG_OPEN_READ_ONLY)
            fail(SLHA_ERR_DIMENSION, "unknown EventLog open mode %d", mode);
        auto L = std::make_unique<EventLogObj>();
        L->writable = mode != SLHA_EVENTLOG_OPEN_READ_ONLY;
        L->fd = ::open(path, (L->writable ? O_RDWR : O_RDONLY) | O_CLOEXEC);
        if (L->fd < 0) io_fail("open");
        struct stat st;
        if (::fstat(L->fd, &st) != 0) io_fail("stat");
        uint64_t len = (uint64_t)st.st_size;
        if (len < kLogHeader) fail(SLHA_ERR_IO, "EventLog: file shorter than header");
        uint8_t h[kLogHeader];
        read_all(L->fd, h, sizeof h, 0);
        if (le32(h) != kLogMagic) fail(SLHA_ERR_IO, "EventLog: bad magic");
        L->version = le32(h + 4);
        if (L->version != kLogV1 && L->version != kLogV2) fail(SLHA_ERR_IO, "EventLog: unsupported version");
        if (le32(h + 8) != 128u) fail(SLHA_ERR_IO, "EventLog: tile-size mismatch");
        const uint64_t rem = (len - kLogHeader) % kLogRecord;
        if (rem != 0) {
            if (mode != SLHA_EVENTLOG_OPEN_RECOVER) fail(SLHA_ERR_IO, "EventLog: truncated record");
            len -= rem;
            if (::ftruncate(L->fd, (off_t)len) != 0) io_fail("truncate");
            if (::fsync(L->fd) != 0) io_fail("sync");
        }
        L->records = (len - kLogHeader) / kLogRecord;
        scan_records(L.get(), [](uint64_t, const uint8_t*) {});
        out = register_log(std::move(L));
    });
    return rc == SLHA_OK ? out : nullptr;
}

int32_t slha_eventlog_append(SlhaEventLog* log, const uint8_t* records, size_t n, int32_t durable) {
    return ffi_status([&] {
        EventLogObj* L = log_of(log);
        std::lock_guard<std::mutex> lock(L->mu);
        if (!L->writable) fail(SLHA_ERR_IO, "EventLog: log opened read-only");
        if (n == 0) return;
        if (!records) fail(SLHA_ERR_NULL, "slha_eventlog_append received a NULL pointer");
        for (size_t i = 0; i < n; ++i) {
            const uint8_t* rec = records + i * kLogRecord;
            const uint32_t want = L->version == kLogV2 ? record_checksum(rec) : 0u;
            if (le32(rec + 12) != want)
                fail(SLHA_ERR_INVALID_TILE, "EventLog: record %zu checksum is not the version-%u value", i,
                     L->version);
        }
        const uint64_t start = kLogHeader + L->records * kLogRecord;
        try {
            write_all(L->fd, records, n * kLogRecord, start);
            if (durable && ::fsync(L->fd) != 0) io_fail("sync");
        } catch (...) {
            if (::ftruncate(L->fd, (off_t)start) == 0 && durable) (void)::fsync(L->fd);
            throw;
        }
        L->records += n;
    });
}

int32_t slha_eventlog_sync(SlhaEventLog* log) {
    return ffi_status([&] {
        EventLogObj* L = log_of(log);
        std::lock_guard<std::mutex> lock(L->mu);
        if (L->writable && ::fsync(L->fd) != 0) io_fail("sync");
    });
}

uint64_t slha_eventlog_len(const SlhaEventLog* log) {
    uint64_t n = 0;
    const int32_t rc = ffi_status([&] {
        EventLogObj* L = log_of(log);
        std::lock_guard<std::mutex> lock(L->mu);
        n = L->records;
    });
    return rc == SLHA_OK ? n : 0;
}

uint32_t slha_eventlog_version(const SlhaEventLog* log) {
    uint32_t v = 0;
    const int32_t rc = ffi_status([&] { v = log_of(log)->version; });
    return rc == SLHA_OK ? v : 0;
}

int32_t slha_eventlog_read(SlhaEventLog* log, uint64_t first, size_t n, uint8_t* records_out) {
    return ffi_status([&] {
        EventLogObj* L = log_of(log);
        std::lock_guard<std::mutex> lock(L->mu);
        if (first > L->records || n > L->records - first)
            fail(SLHA_ERR_DIMENSION, "EventLog: records [%llu, %llu) out of range (len %llu)",
                 (unsigned long long)first, (unsigned long long)(first + n),
                 (unsigned long long)L->records);
        if (n == 0) return;
        if (!records_out) fail(SLHA_ERR_NULL, "slha_eventlog_read received a NULL pointer");
        read_all(L->fd, records_out, n * kLogRecord, kLogHeader + first * kLogRecord);
        for (size_t i = 0; i < n; ++i)
            if (!record_ok(records_out + i * kLogRecord, L->version))
                fail(SLHA_ERR_IO, "EventLog: record checksum mismatch");
    });
}

static int32_t find_latest(SlhaEventLog* log, uint64_t* index_out, int32_t* found,
                           bool (*match)(const uint8_t*, uint64_t), uint64_t key) {
    return ffi_status([&] {
        if (!index_out || !found) fail(SLHA_ERR_NULL, "EventLog lookup received a NULL pointer");
        EventLogObj* L = log_of(log);
        std::lock_guard<std::mutex> lock(L->mu);
        bool hit = false;
        uint64_t at = 0;
        scan_records(L, [&](uint64_t i, const uint8_t* rec) {
            if (match(rec, key)) hit = true, at = i;
        });
        *found = hit ? 1 : 0;
        *index_out = at;
    });
}

int32_t slha_eventlog_find_seq(SlhaEventLog* log, uint64_t seq, uint64_t* index_out, int32_t* found) {
    return find_latest(log, index_out, found, [](const uint8_t* r, uint64_t k) { return le64(r) == k; }, seq);
}

int32_t slha_eventlog_find_slot(SlhaEventLog* log, uint32_t slot, uint64_t* index_out, int32_t* found) {
    return find_latest(log, index_out, found, [](const uint8_t* r, uint64_t k) { return le32(r + 8) == k; },
                       slot);
}

int32_t slha_eventlog_close(SlhaEventLog* log) {
    return ffi_status([&] {
        if (!log) fail(SLHA_ERR_NULL, "EventLog handle is NULL");
        std::unique_ptr<EventLogObj> obj;
        {
            auto& r = log_registry();
            std::lock_guard<std::mutex> lock(r.mu);
            auto it = r.live.find(reinterpret_cast<uintptr_t>(log));
            if (it == r.live.end()) fail(SLHA_ERR_INVALID_HANDLE, "EventLog handle is not a live SLHA handle");
            obj = std::move(it->second);
            r.live.erase(it);
        }
        std::lock_guard<std::mutex> lock(obj->mu);  // waits for a call in flight
    });
}

int32_t slha_gpu_eventlog_pack(const SciRustSlhaTile* arena_dev, const uint32_t* slots_dev,
                               const uint64_t* seqs_dev, size_t n, uint32_t version,
                               uint8_t* records_dev, void* stream) {
    return ffi_status([&] {
        if (version != kLogV1 && version != kLogV2)
            fail(SLHA_ERR_DIMENSION, "EventLog version %u is not 1 or 2", version);
        if (n > ((uint64_t)INT32_MAX) * 256u) fail(SLHA_ERR_DIMENSION, "n=%zu records out of range", n);
        if (n == 0) return;
        if (!arena_dev || !slots_dev || !seqs_dev || !records_dev)
            fail(SLHA_ERR_NULL, "slha_gpu_eventlog_pack received a NULL pointer");
        if (reinterpret_cast<uintptr_t>(records_dev) % 16 != 0)
            fail(SLHA_ERR_DIMENSION, "records_dev must be 16-byte aligned");
        require_device();
        check_hip(launch_eventlog_pack(arena_dev, slots_dev, seqs_dev, n, version, records_dev,
                                       static_cast<hipStream_t>(stream)),
                  "eventlog pack kernel");
    });
}

int32_t slha_gpu_eventlog_unpack(const uint8_t* records_dev, size_t n, uint32_t version,
                                 const uint32_t* dst_slots_dev, SciRustSlhaTile* arena_dev,
                                 uint32_t* status_dev, void* stream) {
    return ffi_status([&] {
        if (version != kLogV1 && version != kLogV2)
            fail(SLHA_ERR_DIMENSION, "EventLog version %u is not 1 or 2", version);
        if (n > ((uint64_t)INT32_MAX) * 256u) fail(SLHA_ERR_DIMENSION, "n=%zu records out of range", n);
        if (n == 0) return;
        if (!records_dev || !dst_slots_dev || !arena_dev || !status_dev)
            fail(SLHA_ERR_NULL, "slha_gpu_eventlog_unpack received a NULL pointer");
        if (reinterpret_cast<uintptr_t>(records_dev) % 16 != 0)
            fail(SLHA_ERR_DIMENSION, "records_dev must be 16-byte aligned");
        require_device();
        check_hip(launch_eventlog_unpack(records_dev, n, version, dst_slots_dev, arena_dev, status_dev,
                                         static_cast<hipStream_t>(stream)),
                  "eventlog unpack kernel");
    });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// CCOS ElasticKvCache (scirust/src/ccos.rs) over a device arena: the control
// plane on the host, the byte changes and the importance on the device.

namespace {

constexpr uint8_t kHot = SLHA_CCOS_HOT, kWarm = SLHA_CCOS_WARM, kCold = SLHA_CCOS_COLD;
constexpr uint64_t kHotBytes = 128, kWarmBytes = 96;  // ccos.rs:32-34

struct DevBuf {  // grow-only device staging
    void* p = nullptr;
    size_t cap = 0;
    void* get(size_t bytes) {
        if (bytes > cap) {
            if (p) (void)hipFree(p);
            p = nullptr;
            cap = 0;
            check_hip(hipMalloc(&p, bytes), "hipMalloc (CCOS staging)");
            cap = bytes;
        }
        return p;
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

struct CcosObj {
    uint4* arena = nullptr;
    uint64_t capacity = 0, budget = 0, sink_window = 0;
    int page_policy = 0, evict_policy = 0;
    // host mirror, per slot of the arena prefix
    std::vector<uint8_t> state;
    std::vector<uint64_t> seq;
    std::vector<float> sigma;
    std::vector<uint32_t> position;
    std::vector<uint16_t> flags;
    std::vector<uint32_t> free_list;
    uint64_t live = 0, next_seq = 0, log_errors = 0, blocked = 0;
    SlhaEventLog* log = nullptr;
    bool durable = false;
    // device
    float* importance = nullptr;
    uint8_t* state_dev = nullptr;
    float* obs_ws = nullptr;
    DevBuf stage_a, stage_b, stage_c;
    ~CcosObj() {
        if (importance) (void)hipFree(importance);
        if (state_dev) (void)hipFree(state_dev);
        if (obs_ws) (void)hipFree(obs_ws);
    }
    uint64_t len() const { return state.size(); }
    uint64_t sep_bytes(uint64_t s) const {  // tile.rs:120-128
        return (flags[s] & SLHA_FLAG_TQ3) ? 16 : ((flags[s] & SLHA_FLAG_MIX3) ? 14 : 0);
    }
    uint64_t slot_live_bytes(uint64_t s) const {  // ccos.rs:470-482
        if (state[s] == kCold) return 0;
        const uint64_t base = state[s] == kHot ? kHotBytes : kWarmBytes;
        return base - ((flags[s] & SLHA_FLAG_TQ3_NOCORR) ? sep_bytes(s) : 0);
    }
};

struct CcosRegistry {
    std::mutex mu;
    std::unordered_map<uintptr_t, std::unique_ptr<CcosObj>> live;
};

CcosRegistry& ccos_registry() {
    static CcosRegistry* r = new CcosRegistry();
    return *r;
}

CcosObj* ccos_of(const SlhaCcos* c) {
    if (!c) fail(SLHA_ERR_NULL, "CCOS handle is NULL");
    auto& r = ccos_registry();
    std::lock_guard<std::mutex> lock(r.mu);
    auto it = r.live.find(reinterpret_cast<uintptr_t>(c));
    if (it == r.live.end()) fail(SLHA_ERR_INVALID_HANDLE, "CCOS handle is not a live SLHA handle");
    return it->second.get();
}

// f32::total_cmp as a signed integer key.
int32_t total_key(float f) {
    int32_t k;
    std::memcpy(&k, &f, 4);
    return k ^ (int32_t)((uint32_t)(k >> 31) >> 1);
}

template <class T>
T* stage(DevBuf& b, const T* host, size_t n, hipStream_t s) {
    T* d = static_cast<T*>(b.get(std::max<size_t>(n, 1) * sizeof(T)));
    check_hip(hipMemcpyAsync(d, host, n * sizeof(T), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
    return d;
}

// ccos.rs:497-512
std::vector<uint32_t> paging_order(const CcosObj* C, uint8_t st) {
    std::vector<uint32_t> v;
    for (uint64_t s = 0; s < C->len(); ++s)
        if (C->state[s] == st) v.push_back((uint32_t)s);
    if (C->page_policy == SLHA_CCOS_PAGE_LOWEST_IMPACT_FIRST)
        std::stable_sort(v.begin(), v.end(), [&](uint32_t a, uint32_t b) {
            return total_key(C->sigma[a]) < total_key(C->sigma[b]);
        });
    else
        std::stable_sort(v.begin(), v.end(), [&](uint32_t a, uint32_t b) { return C->seq[a] < C->seq[b]; });
    return v;
}

// The device side of op 0 page_out, 1 drop_correction or 2 evict over
// `slots`: tile bytes and the device copy of each slot's state, in one
// launch (the slot is a kernel argument when there is one), then the
// stream is drained, so the call returns with its work done.
void apply_op(CcosObj* C, const std::vector<uint32_t>& slots, int op, hipStream_t s) {
    if (slots.empty()) return;
    const uint32_t* d = slots.size() == 1 ? nullptr : stage(C->stage_a, slots.data(), slots.size(), s);
    check_hip(launch_ccos_apply(C->arena, C->state_dev, d, slots[0], slots.size(), op, s), "ccos kernel");
    check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
}

// drop_correction's host effect (ccos.rs:386-397); true when bytes were reclaimed.
bool drop_corr_host(CcosObj* C, uint32_t s) {
    const uint64_t n = C->sep_bytes(s);
    if (C->state[s] == kCold || n == 0 || (C->flags[s] & SLHA_FLAG_TQ3_NOCORR)) return false;
    C->flags[s] |= SLHA_FLAG_TQ3_NOCORR;
    C->live -= n;
    return true;
}

// page_out's host effect (ccos.rs:369-378).
bool page_out_host(CcosObj* C, uint32_t s) {
    if (C->state[s] != kHot) return false;
    C->live -= C->slot_live_bytes(s);
    C->flags[s] |= SLHA_FLAG_WARM;
    C->state[s] = kWarm;
    C->live += C->slot_live_bytes(s);
    return true;
}

// The eviction records of `slots` (seq, slot, tile; ccos.rs:410-420),
// packed on the GPU and appended to the attached log in one call. Returns the
// append's status; a failed append leaves the log as it was.
int32_t append_evictions(CcosObj* C, const std::vector<uint32_t>& slots, hipStream_t s) {
    const size_t n = slots.size();
    std::vector<uint64_t> seqs(n);
    for (size_t i = 0; i < n; ++i) seqs[i] = C->seq[slots[i]];
    const uint32_t* ds = stage(C->stage_a, slots.data(), n, s);
    const uint64_t* dq = stage(C->stage_b, seqs.data(), n, s);
    void* dr = C->stage_c.get(n * SLHA_EVENTLOG_RECORD_BYTES);
    const uint32_t version = slha_eventlog_version(C->log);
    if (version == 0) fail(SLHA_ERR_INVALID_HANDLE, "attached EventLog handle is no longer live");
    check_hip(launch_eventlog_pack(C->arena, ds, dq, n, version, dr, s), "eventlog pack kernel");
    std::vector<uint8_t> rec(n * SLHA_EVENTLOG_RECORD_BYTES);
    check_hip(hipMemcpyAsync(rec.data(), dr, rec.size(), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
    return slha_eventlog_append(C->log, rec.data(), n, C->durable ? 1 : 0);
}

// The slots become COLD and go to the free list (ccos.rs:433-436).
void mark_cold(CcosObj* C, const std::vector<uint32_t>& slots, hipStream_t s) {
    for (uint32_t sl : slots) {
        C->live -= C->slot_live_bytes(sl);
        C->state[sl] = kCold;
        C->free_list.push_back(sl);
    }
    apply_op(C, slots, 2, s);
}

// evict (ccos.rs:404-438) of one live slot; true when it became COLD. A
// failed append counts a log error, and under RequireDurable also a blocked
// eviction, and then keeps the slot live.
bool evict_one(CcosObj* C, uint32_t sl, hipStream_t s) {
    if (C->log) {
        if (append_evictions(C, {sl}, s) != SLHA_OK) {
            ++C->log_errors;
            if (C->durable) {
                ++C->blocked;
                return false;
            }
        }
    } else if (C->durable) {
        ++C->blocked;
        return false;
    }
    mark_cold(C, {sl}, s);
    return true;
}

// enforce_budget's last phase (ccos.rs:565-613) over the live slots in
// eviction order: evict while over budget. The prefix whose eviction reaches
// the budget is tried first as one append and one launch. When that append
// fails (the log is left as it was), the slots are taken one at a time as
// the reference takes them, so a failing record costs only itself and, under
// RequireDurable, later slots can still reach the budget.
void evict_in_order(CcosObj* C, const std::vector<uint32_t>& order, hipStream_t s) {
    std::vector<uint32_t> batch;
    uint64_t after = C->live;
    for (uint32_t sl : order) {
        if (after <= C->budget) break;
        after -= C->slot_live_bytes(sl);
        batch.push_back(sl);
    }
    if (batch.empty()) return;
    if (!C->log && !C->durable) return mark_cold(C, batch, s);
    if (C->log && append_evictions(C, batch, s) == SLHA_OK) return mark_cold(C, batch, s);
    for (uint32_t sl : order) {
        if (C->live <= C->budget) break;
        evict_one(C, sl, s);
    }
}

// insert_with_state (ccos.rs:226-247) of tiles already read to the host;
// returns the slots.
std::vector<uint32_t> insert_host(CcosObj* C, const uint8_t* tiles, size_t n) {
    uint64_t fresh = 0;
    const uint64_t reuse = std::min<uint64_t>(n, C->free_list.size());
    fresh = n - reuse;
    if (C->len() + fresh > C->capacity)
        fail(SLHA_ERR_DIMENSION, "CCOS arena full: %llu slots in use, %zu tiles to insert, capacity %llu",
             (unsigned long long)C->len(), n, (unsigned long long)C->capacity);
    std::vector<uint32_t> slots(n);
    for (size_t i = 0; i < n; ++i) {
        const uint8_t* t = tiles + 128 * i;
        float sg;
        std::memcpy(&sg, t + 104, 4);
        uint32_t pos;
        std::memcpy(&pos, t + 112, 4);
        uint16_t fl;
        std::memcpy(&fl, t + 118, 2);
        uint32_t sl;
        if (!C->free_list.empty()) {
            sl = C->free_list.back();
            C->free_list.pop_back();
        } else {
            sl = (uint32_t)C->len();
            C->state.push_back(kCold);
            C->seq.push_back(0);
            C->sigma.push_back(0.0f);
            C->position.push_back(0);
            C->flags.push_back(0);
        }
        C->state[sl] = (fl & SLHA_FLAG_WARM) ? kWarm : kHot;
        C->seq[sl] = C->next_seq++;
        C->sigma[sl] = sg;
        C->position[sl] = pos;
        C->flags[sl] = fl;
        C->live += C->slot_live_bytes(sl);
        slots[i] = sl;
    }
    return slots;
}

}  // namespace

extern "C" {

SlhaCcos* slha_ccos_new(SciRustSlhaTile* arena_dev, size_t capacity, size_t budget_bytes,
                        int32_t page_policy, int32_t eviction_policy, size_t sink_window) {
    SlhaCcos* out = nullptr;
    const int32_t rc = ffi_status([&] {
        if (!arena_dev) fail(SLHA_ERR_NULL, "slha_ccos_new received a NULL arena");
        if (capacity == 0 || capacity > 0xFFFFFFFFull) fail(SLHA_ERR_DIMENSION, "capacity=%zu out of range", capacity);
        if (page_policy != SLHA_CCOS_PAGE_LOWEST_IMPACT_FIRST && page_policy != SLHA_CCOS_PAGE_OLDEST_FIRST)
            fail(SLHA_ERR_DIMENSION, "unknown page-out policy %d", page_policy);
        if (eviction_policy != SLHA_CCOS_EVICT_CAUSAL && eviction_policy != SLHA_CCOS_EVICT_IMPORTANCE)
            fail(SLHA_ERR_DIMENSION, "unknown eviction policy %d", eviction_policy);
        require_device();
        auto C = std::make_unique<CcosObj>();
        C->arena = reinterpret_cast<uint4*>(arena_dev);
        C->capacity = capacity;
        C->budget = budget_bytes;
        C->page_policy = page_policy;
        C->evict_policy = eviction_policy;
        C->sink_window = sink_window;
        check_hip(hipMalloc(reinterpret_cast<void**>(&C->importance), capacity * sizeof(float)), "hipMalloc");
        check_hip(hipMalloc(reinterpret_cast<void**>(&C->state_dev), capacity), "hipMalloc");
        check_hip(hipMalloc(reinterpret_cast<void**>(&C->obs_ws), observe_workspace_floats() * sizeof(float)),
                  "hipMalloc");
        SlhaCcos* token = reinterpret_cast<SlhaCcos*>(new uint64_t(0));
        auto& r = ccos_registry();
        std::lock_guard<std::mutex> lock(r.mu);
        r.live.emplace(reinterpret_cast<uintptr_t>(token), std::move(C));
        out = token;
    });
    return rc == SLHA_OK ? out : nullptr;
}

int32_t slha_ccos_free(SlhaCcos* c) {
    return ffi_status([&] {
        if (!c) fail(SLHA_ERR_NULL, "CCOS handle is NULL");
        std::unique_ptr<CcosObj> obj;
        auto& r = ccos_registry();
        {
            std::lock_guard<std::mutex> lock(r.mu);
            auto it = r.live.find(reinterpret_cast<uintptr_t>(c));
            if (it == r.live.end()) fail(SLHA_ERR_INVALID_HANDLE, "CCOS handle is not a live SLHA handle");
            obj = std::move(it->second);
            r.live.erase(it);
        }
    });
}

int32_t slha_ccos_attach_event_log(SlhaCcos* c, SlhaEventLog* log, int32_t durable) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        if (log) (void)log_of(log);
        C->log = log;
        C->durable = log && durable;
    });
}

int32_t slha_ccos_insert(SlhaCcos* c, const SciRustSlhaTile* tiles_dev, size_t n, uint32_t* slots_out,
                         void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        if (n == 0) return;
        if (!tiles_dev || !slots_out) fail(SLHA_ERR_NULL, "slha_ccos_insert received a NULL pointer");
        const hipStream_t s = static_cast<hipStream_t>(stream);
        std::vector<uint8_t> host(n * 128);
        check_hip(hipMemcpyAsync(host.data(), tiles_dev, host.size(), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        const std::vector<uint32_t> slots = insert_host(C, host.data(), n);
        const uint32_t* d = stage(C->stage_a, slots.data(), n, s);
        check_hip(launch_tile_scatter(tiles_dev, d, n, C->arena, C->importance, C->state_dev, s),
                  "tile scatter kernel");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        std::memcpy(slots_out, slots.data(), n * sizeof(uint32_t));
    });
}

int32_t slha_ccos_observe_scores(SlhaCcos* c, const float* scores_dev, size_t n, float temperature,
                                 void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        if (n > C->len()) fail(SLHA_ERR_DIMENSION, "n=%zu scores for %llu slots", n, (unsigned long long)C->len());
        if (n == 0 || !std::isfinite(temperature) || temperature <= 0.0f) return;
        if (!scores_dev) fail(SLHA_ERR_NULL, "slha_ccos_observe_scores received a NULL pointer");
        const hipStream_t s = static_cast<hipStream_t>(stream);
        // Stream-ordered, no synchronisation: importance and the workspace
        // stay on the device, and every later call that reads them (evict
        // ordering, slha_ccos_slots) copies them on its stream and waits.
        check_hip(launch_observe_scores(scores_dev, C->state_dev, n, temperature, C->importance, C->obs_ws, s),
                  "observe kernels");
    });
}

int32_t slha_ccos_enforce_budget(SlhaCcos* c, int32_t* within_out, void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        auto within = [&] { return C->live <= C->budget; };
        auto finish = [&] {
            if (within_out) *within_out = within() ? 1 : 0;
        };
        if (within()) return finish();
        // Phases 1-3 (ccos.rs:533-563): the host takes each rung in order while
        // over budget; each phase's tiles change in one launch.
        const struct {
            uint8_t st;
            int op;
        } phases[3] = {{kHot, 1}, {kHot, 0}, {kWarm, 1}};
        for (const auto& ph : phases) {
            std::vector<uint32_t> batch;
            for (uint32_t sl : paging_order(C, ph.st)) {
                if (within()) break;
                if (ph.op == 1 ? drop_corr_host(C, sl) : page_out_host(C, sl)) batch.push_back(sl);
            }
            apply_op(C, batch, ph.op, s);
            if (within()) return finish();
        }
        // Phase 4 (ccos.rs:565-613): eviction order.
        std::vector<uint32_t> live;
        for (uint64_t sl = 0; sl < C->len(); ++sl)
            if (C->state[sl] != kCold) live.push_back((uint32_t)sl);
        if (C->evict_policy == SLHA_CCOS_EVICT_CAUSAL) {
            std::stable_sort(live.begin(), live.end(), [&](uint32_t a, uint32_t b) { return C->seq[a] < C->seq[b]; });
        } else {
            std::vector<float> imp(C->len());
            check_hip(hipMemcpyAsync(imp.data(), C->importance, imp.size() * 4, hipMemcpyDeviceToHost, s),
                      "hipMemcpyAsync");
            check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
            const uint64_t sw = (uint32_t)C->sink_window;  // `sink_window as u32`
            std::stable_sort(live.begin(), live.end(), [&](uint32_t a, uint32_t b) {
                const bool sa = C->position[a] < sw, sb = C->position[b] < sw;
                if (sa != sb) return !sa;
                const int32_t ka = total_key(imp[a]), kb = total_key(imp[b]);
                if (ka != kb) return ka < kb;
                return C->seq[a] < C->seq[b];
            });
        }
        evict_in_order(C, live, s);
        finish();
    });
}

int32_t slha_ccos_page_out(SlhaCcos* c, uint32_t slot, void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        if (slot >= C->len()) fail(SLHA_ERR_DIMENSION, "slot %u out of range", slot);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        if (page_out_host(C, slot)) apply_op(C, {slot}, 0, s);
    });
}

int32_t slha_ccos_drop_correction(SlhaCcos* c, uint32_t slot, int32_t* done_out, void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        if (slot >= C->len()) fail(SLHA_ERR_DIMENSION, "slot %u out of range", slot);
        const bool done = drop_corr_host(C, slot);
        if (done) apply_op(C, {slot}, 1, static_cast<hipStream_t>(stream));
        if (done_out) *done_out = done ? 1 : 0;
    });
}

int32_t slha_ccos_evict(SlhaCcos* c, uint32_t slot, int32_t* done_out, void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        bool done = false;
        if (slot < C->len() && C->state[slot] != kCold) done = evict_one(C, slot, static_cast<hipStream_t>(stream));
        if (done_out) *done_out = done ? 1 : 0;
    });
}

int32_t slha_ccos_rehydrate(SlhaCcos* c, uint64_t seq, int64_t* slot_out, void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        if (!slot_out) fail(SLHA_ERR_NULL, "slha_ccos_rehydrate received a NULL pointer");
        *slot_out = -1;
        if (!C->log) return;
        uint64_t idx = 0;
        int32_t found = 0;
        if (slha_eventlog_find_seq(C->log, seq, &idx, &found) != SLHA_OK)
            fail(SLHA_ERR_IO, "%s", slha_last_error_message());
        if (!found) return;
        uint8_t rec[SLHA_EVENTLOG_RECORD_BYTES];
        if (slha_eventlog_read(C->log, idx, 1, rec) != SLHA_OK) fail(SLHA_ERR_IO, "%s", slha_last_error_message());
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const std::vector<uint32_t> slots = insert_host(C, rec + 16, 1);
        const uint8_t* dt = stage(C->stage_b, rec + 16, 128, s);
        const uint32_t* d = stage(C->stage_a, slots.data(), 1, s);
        check_hip(launch_tile_scatter(dt, d, 1, C->arena, C->importance, C->state_dev, s), "tile scatter kernel");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        *slot_out = slots[0];
    });
}

int32_t slha_ccos_stats(const SlhaCcos* c, SlhaCcosStats* out) {
    return ffi_status([&] {
        const CcosObj* C = ccos_of(c);
        if (!out) fail(SLHA_ERR_NULL, "slha_ccos_stats received a NULL pointer");
        SlhaCcosStats st{};
        st.live_bytes = C->live;
        st.len = C->len();
        for (uint64_t sl = 0; sl < C->len(); ++sl) {
            const uint8_t x = C->state[sl];
            (x == kHot ? st.hot : x == kWarm ? st.warm : st.cold) += 1;
            if (x != kCold && (C->flags[sl] & SLHA_FLAG_TQ3_NOCORR)) {
                st.nocorr += 1;
                st.reclaimed_correction += C->sep_bytes(sl);
            }
        }
        st.log_errors = C->log_errors;
        st.blocked_evictions = C->blocked;
        *out = st;
    });
}

int32_t slha_ccos_slots(SlhaCcos* c, size_t n, int32_t* state_out, uint64_t* seq_out, float* importance_out,
                        void* stream) {
    return ffi_status([&] {
        CcosObj* C = ccos_of(c);
        if (n > C->len()) fail(SLHA_ERR_DIMENSION, "n=%zu exceeds %llu slots", n, (unsigned long long)C->len());
        for (size_t i = 0; i < n; ++i) {
            if (state_out) state_out[i] = C->state[i];
            if (seq_out) seq_out[i] = C->seq[i];
        }
        if (importance_out && n) {
            const hipStream_t s = static_cast<hipStream_t>(stream);
            check_hip(hipMemcpyAsync(importance_out, C->importance, n * 4, hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
            check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        }
    });
}

}  // extern "C"
