// C-ABI layer of libspaceslug_runtime.so (declarations and contracts in
// include/runtime_abi.h). Host C++ calling HIP directly: argument validation
// first (so contract violations return 1 without touching a device), then
// per-device state, staging of host buffers, the kernel launch and, for the
// synchronous entry points, the copy back. Every HIP failure and every C++
// exception is turned into status 2 with a message in spaceslug_last_error();
// the int4 path has no CPU implementation, so without a HIP device every
// compute entry point returns 2.
#include "runtime_abi.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <atomic>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "cq4_kernels.hpp"
#include "q4_kernels.hpp"

static_assert(spaceslug::kMaxLoraRank == SPACESLUG_Q4_MAX_LORA_RANK, "one LoRA rank limit");

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
    g_last_error = message;
    return code;
}

int ok() {
    g_last_error.clear();
    return SPACESLUG_OK;
}

struct HipError {
    hipError_t code;
    const char* what;
};

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw HipError{e, what};
}

int from_hip(const HipError& e) {
    return fail(SPACESLUG_ERR_DEVICE, std::string(e.what) + ": " + hipGetErrorName(e.code) + " (" +
                                          hipGetErrorString(e.code) + ")");
}

// Device scratch of spaceslug_q4gemm_device_noalloc: a module global, so each device the
// library runs on holds its own copy from module load until the process ends, and no call
// allocates or frees it. In host code `scratch` names a host-side stand-in, never the device
// memory: kernels receive the per-device address that hipGetSymbolAddress returns
// (DeviceState::scratch, queried once per device when the device's state is set up).
constexpr size_t kNoAllocScratchBytes = SPACESLUG_Q4_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// Per-device state: launch-relevant properties, the grow-only workspace of
// the device-pointer entry points and the address of this device's copy of
// `scratch`. ws_done marks the end of the last call that used the workspace, on
// ws_stream; a call on another stream waits for it.
struct DeviceState {
    bool ready = false;
    spaceslug::DeviceInfo info{};
    void* scratch = nullptr;
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    hipEvent_t ws_done = nullptr;
    hipStream_t ws_stream = nullptr;
    bool ws_used = false;
    // Device buffers of the synchronous host-pointer calls (grow-only, reused call after call),
    // and the lock a call holds while it uses them.
    void* staging = nullptr;
    size_t staging_bytes = 0;
    std::mutex staging_mutex;
};

// Fixed table: setting up a device's state allocates nothing on the host either.
constexpr int kMaxDevices = 64;
std::mutex g_device_mutex;
DeviceState g_devices[kMaxDevices];

// Number of visible devices, queried once (the set of devices is fixed for the process). The
// cache is written under g_device_mutex, so threads that race on the first call all see one
// value; a failed query is not cached and is retried by the next call.
int device_count() {
    static std::atomic<int> cached{-1};
    int c = cached.load(std::memory_order_acquire);
    if (c > 0) return c;
    std::lock_guard<std::mutex> lock(g_device_mutex);
    c = cached.load(std::memory_order_relaxed);
    if (c > 0) return c;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) throw HipError{e == hipSuccess ? hipErrorNoDevice : e, "no HIP device"};
    c = count < kMaxDevices ? count : kMaxDevices;
    cached.store(c, std::memory_order_release);
    return c;
}

DeviceState& current_device() {
    const int count = device_count();
    int id = 0;
    check(hipGetDevice(&id), "hipGetDevice");
    if (id < 0 || id >= count) throw HipError{hipErrorInvalidDevice, "device index beyond the library's table"};
    std::lock_guard<std::mutex> lock(g_device_mutex);
    DeviceState& d = g_devices[id];
    if (!d.ready) {
        hipDeviceProp_t prop;
        check(hipGetDeviceProperties(&prop, id), "hipGetDeviceProperties");
        d.info.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;
        d.info.max_lds_bytes = prop.sharedMemPerBlock;
        // this device is current: the address is its own copy of the array
        check(hipGetSymbolAddress(&d.scratch, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (scratch)");
        d.ready = true;
    }
    return d;
}

// Returns the device workspace holding at least `bytes` (the caller holds
// g_device_mutex); growing it waits for the device so no queued kernel still
// reads the old buffer.
void* device_workspace(DeviceState& d, size_t bytes) {
    if (bytes == 0) return nullptr;
    if (d.workspace_bytes < bytes) {
        if (d.workspace) {
            check(hipDeviceSynchronize(), "hipDeviceSynchronize (workspace growth)");
            check(hipFree(d.workspace), "hipFree (workspace)");
            d.workspace = nullptr;
            d.workspace_bytes = 0;
        }
        check(hipMalloc(&d.workspace, bytes), "hipMalloc (workspace)");
        d.workspace_bytes = bytes;
    }
    return d.workspace;
}

// Largest staging the device keeps between host-pointer calls; a call needing more (a one-off
// weight upload or quantization) allocates for itself and frees on return.
constexpr size_t kStagingKeepBytes = size_t{256} << 20;

// The device buffers of one synchronous host-pointer call, carved into 256-byte aligned slices.
// Up to kStagingKeepBytes they are the device's grow-only staging buffer, so a steady sequence of
// such calls (the per-token projections on resident weights, spaceslug_q4gemm_run) allocates
// nothing after the first: every host-pointer call returns only after its last copy back, so the
// buffer is idle between calls. The device's staging lock is held for the call.
class StagingArena {
public:
    explicit StagingArena(const std::vector<size_t>& sizes) : dev_(current_device()), lock_(dev_.staging_mutex) {
        size_t total = 0;
        for (size_t s : sizes) {
            offsets_.push_back(total);
            total += (s + 255) & ~static_cast<size_t>(255);
        }
        if (total == 0) total = 256;
        if (total > kStagingKeepBytes) {
            check(hipMalloc(&own_, total), "hipMalloc (staging)");
            base_ = own_;
            return;
        }
        if (dev_.staging_bytes < total) {
            if (dev_.staging) {
                check(hipFree(dev_.staging), "hipFree (staging)");
                dev_.staging = nullptr;
                dev_.staging_bytes = 0;
            }
            check(hipMalloc(&dev_.staging, total), "hipMalloc (staging)");
            dev_.staging_bytes = total;
        }
        base_ = dev_.staging;
    }
    ~StagingArena() {
        if (own_) (void)hipFree(own_);
    }
    StagingArena(const StagingArena&) = delete;
    StagingArena& operator=(const StagingArena&) = delete;
    template <typename T>
    T* slice(size_t i) const {
        return reinterpret_cast<T*>(static_cast<char*>(base_) + offsets_[i]);
    }

private:
    DeviceState& dev_;
    std::lock_guard<std::mutex> lock_;
    void* own_ = nullptr;
    void* base_ = nullptr;
    std::vector<size_t> offsets_;
};

// Row and column counts stay below 2^31 - 2^16, so that a kernel's int indices past the last row
// or column (a partly filled workgroup or column run reaches at most 2^16 beyond) cannot wrap.
constexpr uint32_t kMaxRowsCols = INT32_MAX - 65535u;

bool dims_ok(uint32_t m, uint32_t n, uint32_t k) {
    return m >= 1 && n >= 1 && k >= 32 && (k % spaceslug::kGroup) == 0 && m <= kMaxRowsCols &&
           n <= kMaxRowsCols && k <= INT32_MAX;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t bytes_x(uint32_t m, uint32_t k) { return static_cast<size_t>(m) * k * sizeof(float); }
size_t bytes_w(uint32_t n, uint32_t k) { return static_cast<size_t>(n) * (k / 2); }
size_t bytes_s(uint32_t n, uint32_t k) { return static_cast<size_t>(n) * (k / spaceslug::kGroup) * sizeof(float); }
size_t bytes_y(uint32_t m, uint32_t n) { return static_cast<size_t>(m) * n * sizeof(float); }

// Shared body of the synchronous host-pointer calls (with or without LoRA, with
// or without pre-resident weights).
int run_host(const float* x, const uint8_t* w, const float* s, const uint8_t* d_w_resident,
             const float* d_s_resident, const float* la, const float* lb, float* y, uint32_t m,
             uint32_t n, uint32_t k, uint32_t rank, float lora_scale) {
    DeviceState& dev = current_device();
    const spaceslug::Q4Plan plan = spaceslug::plan_q4gemm(dev.info, m, n, k, rank);
    const bool stage_w = d_w_resident == nullptr;
    std::vector<size_t> sizes = {bytes_x(m, k), bytes_y(m, n), plan.workspace_bytes,
                                 stage_w ? bytes_w(n, k) : 0, stage_w ? bytes_s(n, k) : 0,
                                 rank ? static_cast<size_t>(k) * rank * sizeof(float) : 0,
                                 rank ? static_cast<size_t>(rank) * n * sizeof(float) : 0};
    StagingArena arena(sizes);
    float* dx = arena.slice<float>(0);
    float* dy = arena.slice<float>(1);
    void* dws = plan.workspace_bytes ? arena.slice<void>(2) : nullptr;
    const uint8_t* dw = d_w_resident;
    const float* ds = d_s_resident;
    if (stage_w) {
        check(hipMemcpy(arena.slice<uint8_t>(3), w, bytes_w(n, k), hipMemcpyHostToDevice), "hipMemcpy (weights)");
        check(hipMemcpy(arena.slice<float>(4), s, bytes_s(n, k), hipMemcpyHostToDevice), "hipMemcpy (scales)");
        dw = arena.slice<uint8_t>(3);
        ds = arena.slice<float>(4);
    }
    float* dla = nullptr;
    float* dlb = nullptr;
    if (rank) {
        dla = arena.slice<float>(5);
        dlb = arena.slice<float>(6);
        check(hipMemcpy(dla, la, static_cast<size_t>(k) * rank * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy (lora_a)");
        check(hipMemcpy(dlb, lb, static_cast<size_t>(rank) * n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy (lora_b)");
    }
    check(hipMemcpy(dx, x, bytes_x(m, k), hipMemcpyHostToDevice), "hipMemcpy (x)");
    check(spaceslug::launch_q4gemm(plan, dev.info, dx, dw, ds, dy, m, n, k, dla, dlb, rank, lora_scale, dws, nullptr),
          "q4gemm launch");
    check(hipMemcpy(y, dy, bytes_y(m, n), hipMemcpyDeviceToHost), "hipMemcpy (y)");
    return ok();
}

// The event that orders workspace users across streams of one device. It only orders GPU work on
// that device (hipStreamWaitEvent), so it is recorded without the system-scope memory fence a
// default event performs on completion, which cost several microseconds of stream time per call.
void create_ws_event(DeviceState& dev) {
    check(hipEventCreateWithFlags(&dev.ws_done, hipEventDisableTiming | hipEventDisableSystemFence),
          "hipEventCreateWithFlags");
}

// Returns SPACESLUG_ERR_UNSUPPORTED (with a message) when `st` is being captured into a graph,
// else 0. For the calls that use the shared, grow-only workspace.
int refuse_capture(hipStream_t st, const char* what) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    check(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
    if (cs == hipStreamCaptureStatusNone) return 0;
    return fail(SPACESLUG_ERR_UNSUPPORTED,
                std::string(what) + ": this call uses the library's shared workspace, which a captured graph must "
                                    "not hold (a later, larger call may replace it); capture a "
                                    "spaceslug_q4_chain instead, or use spaceslug_q4gemm_device_noalloc");
}

int run_device(const float* dx, const uint8_t* dw, const float* ds, const float* dla, const float* dlb,
               float* dy, uint32_t m, uint32_t n, uint32_t k, uint32_t rank, float lora_scale,
               void* stream) {
    DeviceState& dev = current_device();
    const spaceslug::Q4Plan plan = spaceslug::plan_q4gemm(dev.info, m, n, k, rank);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (plan.workspace_bytes == 0) {
        check(spaceslug::launch_q4gemm(plan, dev.info, dx, dw, ds, dy, m, n, k, dla, dlb, rank, lora_scale, nullptr,
                                       st),
              "q4gemm launch");
        return ok();
    }
    // A graph captured from this stream would keep the shared workspace's address, which a
    // later, larger call frees: refuse before touching it.
    if (const int rc = refuse_capture(st, "q4gemm")) return rc;
    // Calls that use the shared workspace are ordered across streams: a call on a
    // stream other than the previous user's waits (on the GPU) for that user's end.
    std::lock_guard<std::mutex> lock(g_device_mutex);
    void* dws = device_workspace(dev, plan.workspace_bytes);
    if (!dev.ws_done) create_ws_event(dev);
    if (dev.ws_used && dev.ws_stream != st) check(hipStreamWaitEvent(st, dev.ws_done, 0), "hipStreamWaitEvent");
    check(spaceslug::launch_q4gemm(plan, dev.info, dx, dw, ds, dy, m, n, k, dla, dlb, rank, lora_scale, dws, st),
          "q4gemm launch");
    check(hipEventRecord(dev.ws_done, st), "hipEventRecord");
    dev.ws_stream = st;
    dev.ws_used = true;
    return ok();
}

// -- CQ4 -------------------------------------------------------------------------------------------

// Byte sizes of a CQ4 matrix's arrays (the counts cactus_x86.cpp reads), once its
// shape has been accepted by cq4_problem.
struct Cq4Sizes {
    size_t codebook, scale, norms, packed, signs, perm, rotation;
};

bool pow2(uint32_t v) { return v && !(v & (v - 1)); }

// Returns why the matrix/arguments are not accepted, or nullptr (see runtime_abi.h).
const char* cq4_problem(const spaceslug_cq4_matrix* w, const void* a, uint32_t m, const void* c, Cq4Sizes* sz) {
    if (!w || !a || !c) return "null pointer";
    if (m == 0 || m > 65535) return "need 1 <= m <= 65535";
    if (w->bits == 0 || w->bits > 4) return "bits must be 1..4";
    if (w->K == 0 || w->N == 0 || w->group_size == 0 || w->num_groups == 0) return "zero dimension";
    if (w->K > kMaxRowsCols || w->N > kMaxRowsCols) return "dimension too large (K, N <= 2^31 - 2^16)";
    if (!w->codebook || !w->norms || !w->packed_indices) return "codebook, norms and packed_indices are required";
    const bool orth = (w->flags & SPACESLUG_CQ4_FLAG_ORTHOGONAL) != 0;
    const bool inter = (w->flags & SPACESLUG_CQ4_FLAG_INTERLEAVED_4ROW) != 0;
    if (orth && !w->rotation) return "the orthogonal mode needs a rotation";
    if (!orth && (static_cast<uint64_t>(w->group_size) * w->num_groups != w->K)) return "K must equal group_size * num_groups";
    if (!orth && (!pow2(w->group_size) || w->group_size > 256)) return "group_size must be a power of two <= 256";
    const uint32_t gs = orth ? w->K : w->group_size, ng = orth ? 1 : w->num_groups;
    if (inter && (w->bits != 4 || w->N % 4 || gs % 8)) return "interleaved panels need bits == 4, N % 4 == 0, gs % 8 == 0";
    const size_t pgb = (static_cast<size_t>(gs) * w->bits + 7) / 8;
    sz->codebook = (size_t{1} << w->bits) * 2;
    sz->scale = static_cast<size_t>(w->K) * 2;
    sz->norms = static_cast<size_t>(w->N) * ng * 2;
    sz->packed = static_cast<size_t>(w->N) * ng * pgb;
    sz->signs = orth ? 0 : gs;
    sz->perm = orth ? 0 : static_cast<size_t>(gs) * 4;
    sz->rotation = orth ? static_cast<size_t>(w->K) * w->K * 2 : 0;
    return nullptr;
}

}  // namespace

struct spaceslug_q4_weight {
    int device;
    uint32_t n;
    uint32_t k;
    uint8_t* d_packed;
    float* d_scales;
};

// A retained chain: the instantiated graph of its steps' launches and the device
// workspace those launches were recorded against (owned by the chain, so a replay
// shares no memory with any other call).
struct spaceslug_q4_chain {
    int device = -1;
    uint32_t steps = 0;
    void* workspace = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

// Validation shared by the device entry points and the chain steps; returns an
// error message, or nullptr when the arguments are acceptable.
const char* device_call_problem(const float* d_x, const uint8_t* d_w_packed, const float* d_w_scales,
                                const float* d_lora_a, const float* d_lora_b, float* d_y, uint32_t m, uint32_t n,
                                uint32_t k, uint32_t rank) {
    if (!d_x || !d_w_packed || !d_w_scales || !d_y) return "null pointer";
    if (!dims_ok(m, n, k)) return "need 1<=m,n<=2^31-2^16, k%32==0";
    if (!aligned(d_x, 16) || !aligned(d_w_packed, 16) || !aligned(d_w_scales, 4) || !aligned(d_y, 4))
        return "misaligned device pointer";
    if (d_lora_a || d_lora_b) {
        if (!d_lora_a || !d_lora_b) return "LoRA needs both factors";
        if (rank == 0 || rank > SPACESLUG_Q4_MAX_LORA_RANK) return "need 1<=rank<=64";
        if (!aligned(d_lora_a, 4) || !aligned(d_lora_b, 4)) return "misaligned device pointer";
    }
    return nullptr;
}

// Releases whatever a partly built chain holds (the device is current).
void chain_release(spaceslug_q4_chain* c) {
    if (c->exec) (void)hipGraphExecDestroy(c->exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    if (c->workspace) (void)hipFree(c->workspace);
    delete c;
}

}  // namespace

extern "C" {

int spaceslug_vector_add(const float* left, const float* right, float* output, size_t count) {
    if (!left || !right || !output) return fail(SPACESLUG_ERR_INVALID, "spaceslug_vector_add: null pointer");
    for (size_t i = 0; i < count; ++i) output[i] = left[i] + right[i];
    return ok();
}

int spaceslug_sgemm(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                    float* max_relative_error) {
    if (!a || !b || !c || !max_relative_error || m == 0 || n == 0 || k == 0 || m % 64 || n % 64 || k % 32 ||
        m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_sgemm: invalid arguments (need m%64, n%64, k%32, non-null)");
    try {
        (void)current_device();
        const size_t ab = static_cast<size_t>(m) * k * sizeof(float);
        const size_t bb = static_cast<size_t>(k) * n * sizeof(float);
        const size_t cb = static_cast<size_t>(m) * n * sizeof(float);
        StagingArena arena({ab, bb, cb});
        check(hipMemcpy(arena.slice<float>(0), a, ab, hipMemcpyHostToDevice), "hipMemcpy (a)");
        check(hipMemcpy(arena.slice<float>(1), b, bb, hipMemcpyHostToDevice), "hipMemcpy (b)");
        check(spaceslug::launch_sgemm(arena.slice<float>(0), arena.slice<float>(1), arena.slice<float>(2), m, n, k,
                                      nullptr),
              "sgemm launch");
        check(hipMemcpy(c, arena.slice<float>(2), cb, hipMemcpyDeviceToHost), "hipMemcpy (c)");
        *max_relative_error = 0.0f;
        return ok();
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_sgemm: unknown exception");
    }
}

const char* spaceslug_q4gemm_capability(void) {
    return "q4gemm-hip-gfx950 group=32 layout=n-major-lsb-nibble "
           "decode=gemv(m=1,k<=32768 or m=2,2048<=k<=16384: x as hex digits, v_dot8_i32_i4, exact group sums, k>4096 split over a workgroup) "
           "small=mfma(m<=32: x as byte digits, v_mfma_i32_32x32x32_i8, exact group sums) "
           "gemm=mfma(m>32: v_mfma_f32_32x32x16_bf16 on 3 exact x limbs, 128x128 tiles with K-split or 64x64 "
           "whole-K tiles; f32 group sums) accumulate=f64-over-groups lora=fused-epilogue(rank<=64) "
           "chain=fixed_shape_retained_hip_graph_replay";
}

const char* spaceslug_last_error(void) { return g_last_error.c_str(); }

int spaceslug_q4gemm(const float* x, const uint8_t* w_packed, const float* w_scales, float* y, uint32_t m,
                     uint32_t n, uint32_t k) {
    if (!x || !w_packed || !w_scales || !y) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm: null pointer");
    if (!dims_ok(m, n, k)) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm: need 1<=m,n<=2^31-2^16, k>=32, k%32==0");
    try {
        return run_host(x, w_packed, w_scales, nullptr, nullptr, nullptr, nullptr, y, m, n, k, 0, 0.0f);
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4gemm: unknown exception");
    }
}

int spaceslug_q4gemm_lora(const float* x, const uint8_t* w_packed, const float* w_scales, const float* lora_a,
                          const float* lora_b, float* y, uint32_t m, uint32_t n, uint32_t k, uint32_t rank,
                          float scale) {
    if (!x || !w_packed || !w_scales || !lora_a || !lora_b || !y)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_lora: null pointer");
    if (!dims_ok(m, n, k) || rank == 0 || rank > SPACESLUG_Q4_MAX_LORA_RANK)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_lora: need 1<=m,n<=2^31-2^16, k%32==0, 1<=rank<=64");
    try {
        return run_host(x, w_packed, w_scales, nullptr, nullptr, lora_a, lora_b, y, m, n, k, rank, scale);
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4gemm_lora: unknown exception");
    }
}

int spaceslug_q4gemm_device(const float* d_x, const uint8_t* d_w_packed, const float* d_w_scales, float* d_y,
                            uint32_t m, uint32_t n, uint32_t k, void* stream) {
    if (!d_x || !d_w_packed || !d_w_scales || !d_y)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_device: null pointer");
    if (!dims_ok(m, n, k)) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_device: need 1<=m,n<=2^31-2^16, k%32==0");
    if (!aligned(d_x, 16) || !aligned(d_w_packed, 16) || !aligned(d_w_scales, 4) || !aligned(d_y, 4))
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_device: misaligned device pointer");
    try {
        return run_device(d_x, d_w_packed, d_w_scales, nullptr, nullptr, d_y, m, n, k, 0, 0.0f, stream);
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4gemm_device: unknown exception");
    }
}

int spaceslug_q4gemm_device_noalloc(const float* d_x, const uint8_t* d_w_packed, const float* d_w_scales,
                                    float* d_y, uint32_t m, uint32_t n, uint32_t k, void* stream) {
    if (const char* why = device_call_problem(d_x, d_w_packed, d_w_scales, nullptr, nullptr, d_y, m, n, k, 0))
        return fail(SPACESLUG_ERR_INVALID, std::string("spaceslug_q4gemm_device_noalloc: ") + why);
    try {
        DeviceState& dev = current_device();
        const spaceslug::Q4Plan plan = spaceslug::plan_q4gemm(dev.info, m, n, k, 0);
        if (plan.workspace_bytes > kNoAllocScratchBytes)
            return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_device_noalloc: this shape needs " +
                                                   std::to_string(plan.workspace_bytes) +
                                                   " bytes of scratch, more than the fixed " +
                                                   std::to_string(kNoAllocScratchBytes));
        // every byte of scratch a call reads was written earlier in that call: nothing to clear
        check(spaceslug::launch_q4gemm(plan, dev.info, d_x, d_w_packed, d_w_scales, d_y, m, n, k, nullptr, nullptr, 0,
                                       0.0f, plan.workspace_bytes ? dev.scratch : nullptr,
                                       static_cast<hipStream_t>(stream)),
              "q4gemm launch (fixed scratch)");
        return ok();
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4gemm_device_noalloc: unknown exception");
    }
}

int spaceslug_q4gemm_lora_device(const float* d_x, const uint8_t* d_w_packed, const float* d_w_scales,
                                 const float* d_lora_a, const float* d_lora_b, float* d_y, uint32_t m, uint32_t n,
                                 uint32_t k, uint32_t rank, float scale, void* stream) {
    if (!d_x || !d_w_packed || !d_w_scales || !d_lora_a || !d_lora_b || !d_y)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_lora_device: null pointer");
    if (!dims_ok(m, n, k) || rank == 0 || rank > SPACESLUG_Q4_MAX_LORA_RANK)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_lora_device: need 1<=m,n<=2^31-2^16, k%32==0, 1<=rank<=64");
    if (!aligned(d_x, 16) || !aligned(d_w_packed, 16) || !aligned(d_w_scales, 4) || !aligned(d_y, 4) ||
        !aligned(d_lora_a, 4) || !aligned(d_lora_b, 4))
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_lora_device: misaligned device pointer");
    try {
        return run_device(d_x, d_w_packed, d_w_scales, d_lora_a, d_lora_b, d_y, m, n, k, rank, scale, stream);
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4gemm_lora_device: unknown exception");
    }
}

spaceslug_q4_weight* spaceslug_q4_weight_create(const uint8_t* w_packed, const float* w_scales, uint32_t n,
                                                uint32_t k) {
    if (!w_packed || !w_scales || !dims_ok(1, n, k)) {
        fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_weight_create: invalid arguments");
        return nullptr;
    }
    spaceslug_q4_weight* h = nullptr;
    try {
        (void)current_device();
        h = new spaceslug_q4_weight{0, n, k, nullptr, nullptr};
        check(hipGetDevice(&h->device), "hipGetDevice");
        check(hipMalloc(reinterpret_cast<void**>(&h->d_packed), bytes_w(n, k)), "hipMalloc (weights)");
        check(hipMalloc(reinterpret_cast<void**>(&h->d_scales), bytes_s(n, k)), "hipMalloc (scales)");
        check(hipMemcpy(h->d_packed, w_packed, bytes_w(n, k), hipMemcpyHostToDevice), "hipMemcpy (weights)");
        check(hipMemcpy(h->d_scales, w_scales, bytes_s(n, k), hipMemcpyHostToDevice), "hipMemcpy (scales)");
        ok();
        return h;
    } catch (const HipError& e) {
        from_hip(e);
    } catch (const std::exception& e) {
        fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4_weight_create: unknown exception");
    }
    spaceslug_q4_weight_destroy(h);
    return nullptr;
}

void spaceslug_q4_weight_destroy(spaceslug_q4_weight* weight) {
    if (!weight) return;
    int prev = -1;
    if (hipGetDevice(&prev) == hipSuccess && prev != weight->device) (void)hipSetDevice(weight->device);
    if (weight->d_packed) (void)hipFree(weight->d_packed);
    if (weight->d_scales) (void)hipFree(weight->d_scales);
    if (prev >= 0 && prev != weight->device) (void)hipSetDevice(prev);
    delete weight;
}

int spaceslug_q4_quantize(const float* w, uint8_t* w_packed, float* w_scales, uint32_t n, uint32_t k) {
    if (!w || !w_packed || !w_scales) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_quantize: null pointer");
    if (!dims_ok(1, n, k) || k / spaceslug::kGroup > 65535u)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_quantize: need n>=1, k>=32, k%32==0, k/32<=65535");
    const size_t count = static_cast<size_t>(n) * k;
    for (size_t i = 0; i < count; ++i)
        if (!std::isfinite(w[i])) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_quantize: non-finite weight");
    try {
        (void)current_device();
        StagingArena arena({count * sizeof(float), bytes_w(n, k), bytes_s(n, k)});
        check(hipMemcpy(arena.slice<float>(0), w, count * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy (w)");
        check(spaceslug::launch_q4_quantize(arena.slice<float>(0), arena.slice<uint8_t>(1), arena.slice<float>(2), n, k,
                                            nullptr),
              "quantize launch");
        check(hipMemcpy(w_packed, arena.slice<uint8_t>(1), bytes_w(n, k), hipMemcpyDeviceToHost), "hipMemcpy (packed)");
        check(hipMemcpy(w_scales, arena.slice<float>(2), bytes_s(n, k), hipMemcpyDeviceToHost), "hipMemcpy (scales)");
        return ok();
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4_quantize: unknown exception");
    }
}

int spaceslug_q4_quantize_device(const float* d_w, uint8_t* d_w_packed, float* d_w_scales, uint32_t n, uint32_t k,
                                 void* stream) {
    if (!d_w || !d_w_packed || !d_w_scales)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_quantize_device: null pointer");
    if (!dims_ok(1, n, k) || k / spaceslug::kGroup > 65535u)
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_quantize_device: need n>=1, k>=32, k%32==0, k/32<=65535");
    if (!aligned(d_w_packed, 16) || !aligned(d_w, 4) || !aligned(d_w_scales, 4))
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_quantize_device: d_w_packed must be 16-byte aligned");
    try {
        (void)current_device();
        check(spaceslug::launch_q4_quantize(d_w, d_w_packed, d_w_scales, n, k, static_cast<hipStream_t>(stream)),
              "quantize launch");
        return ok();
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4_quantize_device: unknown exception");
    }
}

int spaceslug_q4gemm_run(const spaceslug_q4_weight* weight, const float* x, float* y, uint32_t m) {
    if (!weight || !x || !y) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_run: null pointer");
    if (!dims_ok(m, weight->n, weight->k)) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_run: need 1<=m<=2^31-2^16");
    try {
        int cur = -1;
        check(hipGetDevice(&cur), "hipGetDevice");
        if (cur != weight->device)
            return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4gemm_run: weight lives on another device");
        return run_host(x, nullptr, nullptr, weight->d_packed, weight->d_scales, nullptr, nullptr, y, m, weight->n,
                        weight->k, 0, 0.0f);
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4gemm_run: unknown exception");
    }
}

int spaceslug_cq4_matmul(const spaceslug_cq4_matrix* w, const uint16_t* a, uint32_t m, uint16_t* c) {
    Cq4Sizes sz{};
    if (const char* why = cq4_problem(w, a, m, c, &sz))
        return fail(SPACESLUG_ERR_INVALID, std::string("spaceslug_cq4_matmul: ") + why);
    const bool orth = (w->flags & SPACESLUG_CQ4_FLAG_ORTHOGONAL) != 0;
    if (!orth && w->permutation)
        for (uint32_t j = 0; j < w->group_size; ++j)
            if (w->permutation[j] >= w->group_size)
                return fail(SPACESLUG_ERR_INVALID, "spaceslug_cq4_matmul: permutation entry out of range");
    try {
        (void)current_device();
        const size_t a_bytes = static_cast<size_t>(m) * w->K * 2, c_bytes = static_cast<size_t>(m) * w->N * 2;
        const bool has_scale = w->input_scale_recip || w->input_scale;
        const spaceslug::Cq4View shape{w->bits, w->K, w->N, w->group_size, w->num_groups, w->flags};
        StagingArena arena({a_bytes, c_bytes, spaceslug::cq4_workspace_bytes(shape, m), sz.codebook,
                            has_scale ? sz.scale : 0, sz.norms, sz.packed, w->left_signs ? sz.signs : 0,
                            w->right_signs ? sz.signs : 0, w->permutation ? sz.perm : 0, sz.rotation});
        auto up = [&](size_t slot, const void* host, size_t bytes) -> void* {
            if (!host || !bytes) return nullptr;
            void* d = arena.slice<void>(slot);
            check(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice), "hipMemcpy (cq4 input)");
            return d;
        };
        spaceslug::Cq4View v{w->bits, w->K, w->N, w->group_size, w->num_groups, w->flags,
                             static_cast<const uint16_t*>(up(3, w->codebook, sz.codebook)), nullptr, nullptr,
                             static_cast<const uint16_t*>(up(5, w->norms, sz.norms)),
                             static_cast<const uint8_t*>(up(6, w->packed_indices, sz.packed)),
                             orth ? nullptr : static_cast<const int8_t*>(up(7, w->left_signs, sz.signs)),
                             orth ? nullptr : static_cast<const int8_t*>(up(8, w->right_signs, sz.signs)),
                             orth ? nullptr : static_cast<const uint32_t*>(up(9, w->permutation, sz.perm)),
                             orth ? static_cast<const uint16_t*>(up(10, w->rotation, sz.rotation)) : nullptr};
        if (w->input_scale_recip) v.input_scale_recip = static_cast<const uint16_t*>(up(4, w->input_scale_recip, sz.scale));
        else if (w->input_scale) v.input_scale = static_cast<const uint16_t*>(up(4, w->input_scale, sz.scale));
        const uint16_t* da = static_cast<const uint16_t*>(up(0, a, a_bytes));
        check(spaceslug::launch_cq4_matmul(v, da, m, arena.slice<uint16_t>(1), arena.slice<void>(2), nullptr),
              "cq4 launch");
        check(hipMemcpy(c, arena.slice<uint16_t>(1), c_bytes, hipMemcpyDeviceToHost), "hipMemcpy (cq4 output)");
        return ok();
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_cq4_matmul: unknown exception");
    }
}

int spaceslug_cq4_matmul_device(const spaceslug_cq4_matrix* w, const uint16_t* d_a, uint32_t m, uint16_t* d_c,
                                void* stream) {
    Cq4Sizes sz{};
    if (const char* why = cq4_problem(w, d_a, m, d_c, &sz))
        return fail(SPACESLUG_ERR_INVALID, std::string("spaceslug_cq4_matmul_device: ") + why);
    if (!aligned(d_a, 2) || !aligned(d_c, 2) || !aligned(w->packed_indices, 4) || !aligned(w->norms, 2) ||
        !aligned(w->codebook, 2) || (w->permutation && !aligned(w->permutation, 4)))
        return fail(SPACESLUG_ERR_INVALID, "spaceslug_cq4_matmul_device: misaligned device pointer");
    const bool orth = (w->flags & SPACESLUG_CQ4_FLAG_ORTHOGONAL) != 0;
    spaceslug::Cq4View v{w->bits, w->K, w->N, w->group_size, w->num_groups, w->flags, w->codebook,
                         w->input_scale_recip ? nullptr : w->input_scale, w->input_scale_recip, w->norms,
                         w->packed_indices, orth ? nullptr : w->left_signs, orth ? nullptr : w->right_signs,
                         orth ? nullptr : w->permutation, orth ? w->rotation : nullptr};
    try {
        DeviceState& dev = current_device();
        const hipStream_t st = static_cast<hipStream_t>(stream);
        const size_t ws_bytes = spaceslug::cq4_workspace_bytes(v, m);
        if (ws_bytes == 0) {  // one launch, no workspace (decode sizes): capturable
            check(spaceslug::launch_cq4_matmul(v, d_a, m, d_c, nullptr, st), "cq4 launch");
            return ok();
        }
        if (const int rc = refuse_capture(st, "spaceslug_cq4_matmul_device")) return rc;
        std::lock_guard<std::mutex> lock(g_device_mutex);
        void* ws = device_workspace(dev, ws_bytes);
        if (!dev.ws_done) create_ws_event(dev);
        if (dev.ws_used && dev.ws_stream != st) check(hipStreamWaitEvent(st, dev.ws_done, 0), "hipStreamWaitEvent");
        check(spaceslug::launch_cq4_matmul(v, d_a, m, d_c, ws, st), "cq4 launch");
        check(hipEventRecord(dev.ws_done, st), "hipEventRecord");
        dev.ws_stream = st;
        dev.ws_used = true;
        return ok();
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_cq4_matmul_device: unknown exception");
    }
}

spaceslug_q4_chain* spaceslug_q4_chain_create(const spaceslug_q4_step* steps, uint32_t count) {
    if (!steps || count == 0) {
        fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_chain_create: need at least one step");
        return nullptr;
    }
    for (uint32_t i = 0; i < count; ++i) {
        const spaceslug_q4_step& s = steps[i];
        if (const char* why = device_call_problem(s.d_x, s.d_w_packed, s.d_w_scales, s.d_lora_a, s.d_lora_b, s.d_y,
                                                  s.m, s.n, s.k, s.rank)) {
            fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_chain_create: step " + std::to_string(i) + ": " + why);
            return nullptr;
        }
    }
    spaceslug_q4_chain* c = nullptr;
    hipStream_t capture = nullptr;
    bool capturing = false;
    try {
        DeviceState& dev = current_device();
        c = new spaceslug_q4_chain;
        check(hipGetDevice(&c->device), "hipGetDevice");
        c->steps = count;
        std::vector<spaceslug::Q4Plan> plans;
        size_t ws = 0;
        for (uint32_t i = 0; i < count; ++i) {
            const spaceslug_q4_step& s = steps[i];
            plans.push_back(spaceslug::plan_q4gemm(dev.info, s.m, s.n, s.k, s.d_lora_a ? s.rank : 0));
            ws = std::max(ws, plans.back().workspace_bytes);
        }
        // The steps run one after another inside the graph, so one workspace serves all of them.
        if (ws) check(hipMalloc(&c->workspace, ws), "hipMalloc (chain workspace)");
        check(hipStreamCreateWithFlags(&capture, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        check(hipStreamBeginCapture(capture, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        capturing = true;
        for (uint32_t i = 0; i < count; ++i) {
            const spaceslug_q4_step& s = steps[i];
            const bool lora = s.d_lora_a != nullptr;
            check(spaceslug::launch_q4gemm(plans[i], dev.info, s.d_x, s.d_w_packed, s.d_w_scales, s.d_y, s.m, s.n, s.k,
                                           s.d_lora_a, s.d_lora_b, lora ? s.rank : 0, lora ? s.lora_scale : 0.0f,
                                           c->workspace, capture),
                  "q4gemm launch (capture)");
        }
        capturing = false;
        check(hipStreamEndCapture(capture, &c->graph), "hipStreamEndCapture");
        check(hipGraphInstantiate(&c->exec, c->graph, nullptr, nullptr, 0), "hipGraphInstantiate");
        check(hipStreamDestroy(capture), "hipStreamDestroy");
        capture = nullptr;
        ok();
        return c;
    } catch (const HipError& e) {
        from_hip(e);
    } catch (const std::exception& e) {
        fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4_chain_create: unknown exception");
    }
    if (capturing) {
        hipGraph_t partial = nullptr;
        if (hipStreamEndCapture(capture, &partial) == hipSuccess && partial) (void)hipGraphDestroy(partial);
    }
    if (capture) (void)hipStreamDestroy(capture);
    if (c) chain_release(c);
    return nullptr;
}

int spaceslug_q4_chain_run(spaceslug_q4_chain* chain, void* stream) {
    if (!chain) return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_chain_run: null chain");
    try {
        int cur = -1;
        check(hipGetDevice(&cur), "hipGetDevice");
        if (cur != chain->device)
            return fail(SPACESLUG_ERR_INVALID, "spaceslug_q4_chain_run: chain lives on another device");
        check(hipGraphLaunch(chain->exec, static_cast<hipStream_t>(stream)), "hipGraphLaunch");
        return ok();
    } catch (const HipError& e) {
        return from_hip(e);
    } catch (const std::exception& e) {
        return fail(SPACESLUG_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(SPACESLUG_ERR_DEVICE, "spaceslug_q4_chain_run: unknown exception");
    }
}

void spaceslug_q4_chain_destroy(spaceslug_q4_chain* chain) {
    if (!chain) return;
    const int device = chain->device;
    int prev = -1;
    if (hipGetDevice(&prev) == hipSuccess && prev != device) (void)hipSetDevice(device);
    // a replay still in flight reads the workspace: wait for the device first
    (void)hipDeviceSynchronize();
    chain_release(chain);
    if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
}

}  // extern "C"
