// palladium_hip: hiprtc compile cache, module loading and launches for
// palladium_amd kernels on MI355X (gfx950). C ABI in include/palladium_hip.h.
//
// The kernel cache follows the reference handler's discipline
// (native/ffi/palladium_ffi.cpp:25-91): look up under a mutex, compile
// outside it so different kernels compile concurrently, re-check on
// insert and release the loser of a race.

#include "palladium_hip.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

struct ph_kernel {
  hipModule_t module;
  hipFunction_t function;
  int device;
};

namespace {

char *dup_message(const std::string &s) {
  char *p = static_cast<char *>(std::malloc(s.size() + 1));
  if (p) std::memcpy(p, s.c_str(), s.size() + 1);
  return p;
}

int fail(char **err, int code, const std::string &msg) {
  if (err) *err = dup_message(msg);
  return code;
}

int hip_fail(char **err, hipError_t e, const char *what) {
  return fail(err, PH_ERR_RUNTIME,
              std::string(what) + ": " + hipGetErrorName(e) + " (" +
                  hipGetErrorString(e) + ")");
}

const char *kOptions[4] = {
    "-ffp-contract=off",
    "-ffp-contract=fast",
    "-ffp-contract=fast -ffast-math -fno-finite-math-only -fgpu-flush-denormals-to-zero "
    "-fno-hip-fp32-correctly-rounded-divide-sqrt",
    // REPRODUCIBLE: the emitter writes every fused multiply-add itself.
    "-ffp-contract=off",
};

std::vector<std::string> build_options(int math_mode, const char *arch) {
  std::vector<std::string> o;
  o.push_back(std::string("--offload-arch=") + (arch && *arch ? arch : "gfx950"));
  o.push_back("-O3");
  o.push_back("-std=c++17");
  // Signed integer arithmetic wraps (two's complement), as jnp int32 does;
  // without this an overflowing hash multiply would be undefined behaviour.
  o.push_back("-fwrapv");
  // No SLP vectorisation: with packed FP32 disabled, SLP-packed float16
  // code can reach an instruction-selection failure in the gfx950 backend
  // ("Cannot select: v2f32 = bitcast", an abort inside hiprtc). The hot
  // kernels compile to identical code either way.
  o.push_back("-fno-slp-vectorize");
  // Packed FP32 VALU forms are kept out of every code object.
  o.push_back("-Xclang");
  o.push_back("-target-feature");
  o.push_back("-Xclang");
  o.push_back("-packed-fp32-ops");
  o.push_back("-DPH_MATH_MODE=" + std::to_string(math_mode));
  std::string mode = kOptions[math_mode];
  size_t pos = 0;
  while (pos < mode.size()) {
    size_t sp = mode.find(' ', pos);
    if (sp == std::string::npos) sp = mode.size();
    if (sp > pos) o.push_back(mode.substr(pos, sp - pos));
    pos = sp + 1;
  }
  return o;
}

int compile(const char *src, size_t src_len, const char *name, int math_mode,
            const char *arch, std::vector<char> *code, char **err) {
  if (math_mode < PH_MATH_SAFE || math_mode > PH_MATH_REPRODUCIBLE)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip: math_mode out of range");
  std::string source(src, src_len);
  std::string fname = std::string(name ? name : "kernel") + ".hip";
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source.c_str(), fname.c_str(), 0,
                                       nullptr, nullptr);
  if (r != HIPRTC_SUCCESS)
    return fail(err, PH_ERR_COMPILE,
                std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
  std::vector<std::string> opts = build_options(math_mode, arch);
  std::vector<const char *> copts;
  for (auto &s : opts) copts.push_back(s.c_str());
  r = hiprtcCompileProgram(prog, (int)copts.size(), copts.data());
  if (r != HIPRTC_SUCCESS) {
    size_t log_size = 0;
    hiprtcGetProgramLogSize(prog, &log_size);
    std::string log(log_size, '\0');
    if (log_size) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return fail(err, PH_ERR_COMPILE,
                std::string("hiprtc compile failed (") + hiprtcGetErrorString(r) +
                    "):\n" + log);
  }
  size_t size = 0;
  r = hiprtcGetCodeSize(prog, &size);
  if (r == HIPRTC_SUCCESS) {
    code->resize(size);
    r = hiprtcGetCode(prog, code->data());
  }
  (void)hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS)
    return fail(err, PH_ERR_COMPILE, std::string("hiprtcGetCode: ") + hiprtcGetErrorString(r));
  return PH_OK;
}

class KernelCache {
 public:
  static KernelCache &instance() {
    static KernelCache *cache = new KernelCache();  // never destroyed: modules
    return *cache;                                  // outlive static teardown
  }

  int get(const char *src, size_t src_len, const char *name, int math_mode,
          ph_kernel **out, char **err) {
    int device = 0;
    hipError_t he = hipGetDevice(&device);
    if (he != hipSuccess) return hip_fail(err, he, "hipGetDevice");
    std::string key;
    key.reserve(src_len + 64);
    key.append(src, src_len);
    key.push_back('\0');
    key.append(name);
    key.push_back('\0');
    key.append(std::to_string(math_mode));
    key.push_back('\0');
    key.append(std::to_string(device));
    {
      std::lock_guard<std::mutex> lock(mutex_);
      auto it = entries_.find(key);
      if (it != entries_.end()) {
        *out = it->second.get();
        return PH_OK;
      }
    }
    std::vector<char> code;
    int rc = compile(src, src_len, name, math_mode, "gfx950", &code, err);
    if (rc != PH_OK) return rc;
    auto k = std::make_unique<ph_kernel>();
    k->device = device;
    he = hipModuleLoadData(&k->module, code.data());
    if (he != hipSuccess) return hip_fail(err, he, "hipModuleLoadData");
    he = hipModuleGetFunction(&k->function, k->module, name);
    if (he != hipSuccess) {
      (void)hipModuleUnload(k->module);  // best effort: the lookup error is reported
      return hip_fail(err, he, (std::string("hipModuleGetFunction(") + name + ")").c_str());
    }
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = entries_.find(key);
    if (it != entries_.end()) {
      (void)hipModuleUnload(k->module);  // lost the race: keep the cached module
      *out = it->second.get();
      return PH_OK;
    }
    *out = k.get();
    entries_.emplace(std::move(key), std::move(k));
    return PH_OK;
  }

  size_t size() {
    std::lock_guard<std::mutex> lock(mutex_);
    return entries_.size();
  }

 private:
  std::mutex mutex_;
  std::unordered_map<std::string, std::unique_ptr<ph_kernel>> entries_;
};

}  // namespace

extern "C" {

const char *ph_version(void) { return "0.1.0"; }

void ph_free_error(char *err) { std::free(err); }

int ph_compile_code_object(const char *src, size_t src_len, const char *name,
                           int math_mode, const char *arch, void **code,
                           size_t *code_size, char **err) {
  if (!src || !name || !code || !code_size)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_compile_code_object: null argument");
  std::vector<char> buf;
  int rc = compile(src, src_len, name, math_mode, arch, &buf, err);
  if (rc != PH_OK) return rc;
  void *p = std::malloc(buf.size());
  if (!p) return fail(err, PH_ERR_RUNTIME, "out of host memory");
  std::memcpy(p, buf.data(), buf.size());
  *code = p;
  *code_size = buf.size();
  return PH_OK;
}

void ph_free_code_object(void *code) { std::free(code); }

const char *ph_compile_options(int math_mode) {
  if (math_mode < PH_MATH_SAFE || math_mode > PH_MATH_REPRODUCIBLE) return "";
  return kOptions[math_mode];
}

int ph_get_kernel(const char *src, size_t src_len, const char *name,
                  int math_mode, ph_kernel **out, char **err) {
  if (!src || !name || !out)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_get_kernel: null argument");
  if (math_mode < PH_MATH_SAFE || math_mode > PH_MATH_REPRODUCIBLE)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip: math_mode out of range");
  return KernelCache::instance().get(src, src_len, name, math_mode, out, err);
}

int ph_load_code_object(const void *code, size_t code_size, const char *name,
                        ph_kernel **out, char **err) {
  if (!code || !code_size || !name || !out)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_load_code_object: null argument");
  int device = 0;
  hipError_t he = hipGetDevice(&device);
  if (he != hipSuccess) return hip_fail(err, he, "hipGetDevice");
  auto k = std::make_unique<ph_kernel>();
  k->device = device;
  he = hipModuleLoadData(&k->module, code);
  if (he != hipSuccess) return hip_fail(err, he, "hipModuleLoadData");
  he = hipModuleGetFunction(&k->function, k->module, name);
  if (he != hipSuccess) {
    (void)hipModuleUnload(k->module);  // best effort: the lookup error is reported
    return hip_fail(err, he, (std::string("hipModuleGetFunction(") + name + ")").c_str());
  }
  *out = k.release();  // kept for the life of the process, like cached kernels
  return PH_OK;
}

size_t ph_kernel_cache_size(void) { return KernelCache::instance().size(); }

int ph_launch(ph_kernel *k, unsigned int gx, unsigned int gy, unsigned int gz,
              unsigned int bx, unsigned int by, unsigned int bz,
              unsigned int shared, void *stream, void **params, char **err) {
  if (!k) return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_launch: null kernel");
  if (gx == 0 || gy == 0 || gz == 0 || bx == 0 || by == 0 || bz == 0 ||
      (size_t)bx * by * bz > 1024)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_launch: invalid launch geometry");
  hipError_t e = hipModuleLaunchKernel(k->function, gx, gy, gz, bx, by, bz, shared,
                                       (hipStream_t)stream, params, nullptr);
  if (e != hipSuccess) return hip_fail(err, e, "hipModuleLaunchKernel");
  return PH_OK;
}

int ph_launch_ptrs(ph_kernel *k, unsigned int blocks, unsigned int block,
                   void *stream, void *const *ptrs, size_t n_ptrs, char **err) {
  if (n_ptrs && !ptrs) return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_launch_ptrs: null pointer array");
  std::vector<void *> values(ptrs, ptrs + n_ptrs);
  std::vector<void *> params(n_ptrs);
  for (size_t i = 0; i < n_ptrs; ++i) params[i] = &values[i];
  return ph_launch(k, blocks, 1, 1, block, 1, 1, 0, stream,
                   n_ptrs ? params.data() : nullptr, err);
}

namespace {

// Validate the dispatch attributes and derive the 1-D launch: `lanes`
// threads per program instance (1, or the block rows of a lane-parallel
// kernel), ceil(programs * lanes / block) workgroups. This is the geometry
// the emitter compiled into the source (its XCD remap and bounds guard).
int dispatch_geometry(int64_t grid_x, int64_t grid_y, int64_t grid_z, int64_t block_x,
                      int64_t lanes, int64_t math_mode, unsigned int *blocks,
                      unsigned int *block, char **err) {
  if (math_mode < PH_MATH_SAFE || math_mode > PH_MATH_REPRODUCIBLE)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip_dispatch: math_mode out of range");
  if (grid_x <= 0 || grid_y <= 0 || grid_z <= 0)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip_dispatch: grid dims must be positive");
  if (lanes <= 0 || lanes > 1024)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip_dispatch: lanes must be in [1, 1024]");
  int64_t b = block_x > 0 ? block_x : 256;
  if (b > 1024 || b % 64)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip_dispatch: block must be a multiple of 64, at most 1024");
  if (grid_x >= (int64_t(1) << 31) || grid_y >= (int64_t(1) << 31) || grid_z >= (int64_t(1) << 31))
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip_dispatch: too many program instances");
  int64_t threads = grid_x * grid_y;
  if (threads >= (int64_t(1) << 31) || (threads *= grid_z) >= (int64_t(1) << 31) ||
      (threads *= lanes) >= (int64_t(1) << 31))
    return fail(err, PH_ERR_INVALID_ARGUMENT, "palladium_hip_dispatch: too many program instances");
  *block = (unsigned int)b;
  *blocks = (unsigned int)((threads + b - 1) / b);
  return PH_OK;
}

// Per-thread, per-device staging for host-buffer dispatch: one stream and
// one device buffer per operand slot, grown on demand and reused by every
// later call on that thread, so a dispatch allocates nothing in the steady
// state (hipMalloc/hipFree and stream creation cost tens of microseconds
// each). XLA:CPU calls the handler from its thread pool; thread-local
// staging needs no lock. Kept for the life of the process, like the kernel
// cache.
struct DispatchStaging {
  hipStream_t stream = nullptr;
  std::vector<void *> bufs;
  std::vector<size_t> caps;
  // Pinned host memory small outputs are read back into before the final
  // memcpy: for 16 KB that takes 28 us against 41 us straight into pageable
  // memory; at 1 MB the extra memcpy loses (130 against 117 us), so only
  // outputs up to 64 KiB in total take this way.
  void *bounce = nullptr;
  size_t bounce_cap = 0;
  static constexpr size_t kBounceMax = 64u << 10;

  int reserve_bounce(size_t bytes, char **err) {
    if (bytes <= bounce_cap) return PH_OK;
    if (bounce) (void)hipHostFree(bounce);  // idle: every dispatch ends synchronized
    bounce = nullptr;
    bounce_cap = 0;
    size_t cap = bytes < 65536 ? 65536 : bytes;
    hipError_t e = hipHostMalloc(&bounce, cap, hipHostMallocDefault);
    if (e != hipSuccess) return hip_fail(err, e, "hipHostMalloc");
    bounce_cap = cap;
    return PH_OK;
  }

  int reserve(size_t slot, size_t bytes, char **err) {
    if (slot >= bufs.size()) {
      bufs.resize(slot + 1, nullptr);
      caps.resize(slot + 1, 0);
    }
    if (bytes <= caps[slot] && bufs[slot]) return PH_OK;
    size_t cap = bytes < 256 ? 256 : bytes;
    if (bufs[slot]) (void)hipFree(bufs[slot]);  // grown: the old one is idle
    bufs[slot] = nullptr;
    caps[slot] = 0;
    hipError_t e = hipMalloc(&bufs[slot], cap);
    if (e != hipSuccess) return hip_fail(err, e, "hipMalloc");
    caps[slot] = cap;
    return PH_OK;
  }
};

// Staging objects are owned per thread while it lives and go back to a
// per-device pool when it exits, for the next thread that dispatches: a
// program that keeps starting threads (thread-per-request servers) holds
// at most as many as ran at once. Thread exit makes no HIP call (it may
// come during process teardown); pooled objects are idle because every
// dispatch ends with its stream synchronized.
struct StagingPool {
  std::mutex mutex;
  std::unordered_map<int, std::vector<DispatchStaging *>> idle;
  size_t created = 0;

  static StagingPool &instance() {
    static StagingPool *pool = new StagingPool();  // never destroyed: see above
    return *pool;
  }
};

struct ThreadStaging {
  std::unordered_map<int, DispatchStaging *> per_device;
  ~ThreadStaging() {
    StagingPool &pool = StagingPool::instance();
    std::lock_guard<std::mutex> lock(pool.mutex);
    for (auto &kv : per_device)
      if (kv.second) pool.idle[kv.first].push_back(kv.second);
  }
};

int dispatch_staging(DispatchStaging **out, char **err) {
  thread_local ThreadStaging mine;
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return hip_fail(err, e, "hipGetDevice");
  DispatchStaging *&st = mine.per_device[device];
  if (!st) {
    StagingPool &pool = StagingPool::instance();
    {
      std::lock_guard<std::mutex> lock(pool.mutex);
      auto &idle = pool.idle[device];
      if (!idle.empty()) {
        st = idle.back();
        idle.pop_back();
      }
    }
    if (!st) {
      auto fresh = std::make_unique<DispatchStaging>();
      e = hipStreamCreate(&fresh->stream);
      if (e != hipSuccess) return hip_fail(err, e, "hipStreamCreate");
      st = fresh.release();
      std::lock_guard<std::mutex> lock(pool.mutex);
      ++pool.created;
    }
  }
  *out = st;
  return PH_OK;
}

}  // namespace

int ph_dispatch_device(const char *src, size_t src_len, const char *name,
                       int64_t grid_x, int64_t grid_y, int64_t grid_z, int64_t block_x,
                       int64_t lanes, int64_t math_mode, void *stream,
                       const void *const *inputs, size_t n_inputs,
                       void *const *outputs, size_t n_outputs, char **err) {
  if ((n_inputs && !inputs) || (n_outputs && !outputs))
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_dispatch_device: null operand array");
  unsigned int blocks = 0, block = 0;
  int rc = dispatch_geometry(grid_x, grid_y, grid_z, block_x, lanes, math_mode, &blocks, &block, err);
  if (rc != PH_OK) return rc;
  ph_kernel *k = nullptr;
  rc = ph_get_kernel(src, src_len, name, (int)math_mode, &k, err);
  if (rc != PH_OK) return rc;
  std::vector<void *> ptrs;
  ptrs.reserve(n_inputs + n_outputs);
  for (size_t i = 0; i < n_inputs; ++i) ptrs.push_back(const_cast<void *>(inputs[i]));
  for (size_t i = 0; i < n_outputs; ++i) ptrs.push_back(outputs[i]);
  return ph_launch_ptrs(k, blocks, block, stream, ptrs.data(), ptrs.size(), err);
}

int ph_dispatch(const char *src, size_t src_len, const char *name,
                int64_t grid_x, int64_t grid_y, int64_t grid_z, int64_t block_x,
                int64_t lanes, int64_t math_mode, const void *const *inputs,
                const size_t *input_bytes, size_t n_inputs,
                void *const *outputs, const size_t *output_bytes,
                size_t n_outputs, char **err) {
  if ((n_inputs && (!inputs || !input_bytes)) || (n_outputs && (!outputs || !output_bytes)))
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_dispatch: null operand array");
  unsigned int blocks = 0, block = 0;
  int rc = dispatch_geometry(grid_x, grid_y, grid_z, block_x, lanes, math_mode, &blocks, &block, err);
  if (rc != PH_OK) return rc;
  ph_kernel *k = nullptr;
  rc = ph_get_kernel(src, src_len, name, (int)math_mode, &k, err);
  if (rc != PH_OK) return rc;

  DispatchStaging *st = nullptr;
  rc = dispatch_staging(&st, err);
  if (rc != PH_OK) return rc;
  const size_t n_ops = n_inputs + n_outputs;
  for (size_t i = 0; i < n_ops; ++i) {
    rc = st->reserve(i, i < n_inputs ? input_bytes[i] : output_bytes[i - n_inputs], err);
    if (rc != PH_OK) return rc;
  }
  std::vector<void *> dev(st->bufs.begin(), st->bufs.begin() + n_ops);
  // Once work is queued, every exit drains the staging stream first: a
  // queued copy must not touch the caller's host buffers after we return,
  // nor a staging buffer the next call on this thread regrows.
  auto drain_and = [&](int code) {
    (void)hipStreamSynchronize(st->stream);  // best effort: `code` is the error reported
    return code;
  };
  hipError_t e;
  for (size_t i = 0; i < n_inputs; ++i) {
    if (!input_bytes[i]) continue;
    e = hipMemcpyHtoDAsync(dev[i], const_cast<void *>(inputs[i]), input_bytes[i], st->stream);
    if (e != hipSuccess) return drain_and(hip_fail(err, e, "hipMemcpyHtoDAsync"));
  }
  rc = ph_launch_ptrs(k, blocks, block, st->stream, dev.data(), dev.size(), err);
  if (rc != PH_OK) return drain_and(rc);
  size_t out_total = 0;
  for (size_t i = 0; i < n_outputs; ++i) out_total += output_bytes[i];
  const bool bounce = out_total <= DispatchStaging::kBounceMax;
  if (bounce) {
    rc = st->reserve_bounce(out_total, err);
    if (rc != PH_OK) return drain_and(rc);
  }
  size_t off = 0;
  for (size_t i = 0; i < n_outputs; ++i) {
    if (!output_bytes[i]) continue;
    void *dst = bounce ? static_cast<char *>(st->bounce) + off : outputs[i];
    e = hipMemcpyDtoHAsync(dst, dev[n_inputs + i], output_bytes[i], st->stream);
    if (e != hipSuccess) return drain_and(hip_fail(err, e, "hipMemcpyDtoHAsync"));
    off += output_bytes[i];
  }
  e = hipStreamSynchronize(st->stream);
  if (e == hipSuccess && bounce) {
    off = 0;
    for (size_t i = 0; i < n_outputs; ++i) {
      if (output_bytes[i]) std::memcpy(outputs[i], static_cast<char *>(st->bounce) + off, output_bytes[i]);
      off += output_bytes[i];
    }
  }
  if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
  return PH_OK;
}

size_t ph_dispatch_staging_count(void) {
  StagingPool &pool = StagingPool::instance();
  std::lock_guard<std::mutex> lock(pool.mutex);
  return pool.created;
}

}  // extern "C"

namespace {

// The allocation-free dispatch's staging: one fixed device array per GPU,
// reserved when the library's code object is loaded. In host code
// `scratch` names a host-side stand-in, never device memory; every use
// goes through the per-device address hipGetSymbolAddress returns.
constexpr size_t kScratchBytes = size_t(PH_NOALLOC_SCRATCH_BYTES);
constexpr size_t kScratchAlign = 256;
constexpr int kMaxDevices = 64;
constexpr size_t kMaxOperands = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};
// One lock per device's copy of `scratch`: a call holds it from its first
// copy into the array to the stream synchronisation after its last copy out,
// so calls that overlap on one GPU (threads of one process) run one after
// another instead of overwriting each other's operands. Static storage, no
// allocation.
std::mutex g_scratch_use[kMaxDevices];

// Looks up this device's copy of `scratch` once, with the device current.
int scratch_address(int device, void **out, char **err) {
  if (device < 0 || device >= kMaxDevices)
    return fail(err, PH_ERR_RUNTIME, "ph_dispatch_noalloc: device ordinal beyond 64");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(err, e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(err, PH_ERR_RUNTIME, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return PH_OK;
}

// Zero `words` 32-bit words from `p` (grid-stride). A kernel, not
// hipMemsetAsync, so the clear stays an ordinary kernel node wherever the
// caller's stream is.
__global__ void __launch_bounds__(256) zero_words(uint32_t *p, size_t words) {
  size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride) p[i] = 0u;
}

size_t align_up(size_t x) { return (x + kScratchAlign - 1) / kScratchAlign * kScratchAlign; }

}  // namespace

extern "C" {

size_t ph_noalloc_scratch_bytes(void) { return kScratchBytes; }

int ph_dispatch_noalloc(ph_kernel *k, int64_t grid_x, int64_t grid_y, int64_t grid_z,
                        int64_t block_x, int64_t lanes, void *stream,
                        const void *const *inputs, const size_t *input_bytes, size_t n_inputs,
                        void *const *outputs, const size_t *output_bytes, size_t n_outputs,
                        char **err) {
  if (!k) return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_dispatch_noalloc: null kernel");
  if ((n_inputs && (!inputs || !input_bytes)) || (n_outputs && (!outputs || !output_bytes)))
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_dispatch_noalloc: null operand array");
  const size_t n_ops = n_inputs + n_outputs;
  if (n_inputs > kMaxOperands || n_outputs > kMaxOperands || n_ops > kMaxOperands)
    return fail(err, PH_ERR_INVALID_ARGUMENT, "ph_dispatch_noalloc: more than 64 operands");
  unsigned int blocks = 0, block = 0;
  int rc = dispatch_geometry(grid_x, grid_y, grid_z, block_x, lanes, PH_MATH_SAFE, &blocks, &block, err);
  if (rc != PH_OK) return rc;
  // Place every operand at a 256-byte boundary; reject what does not fit.
  size_t offs[kMaxOperands];
  size_t total = 0;
  for (size_t i = 0; i < n_ops; ++i) {
    size_t b = i < n_inputs ? input_bytes[i] : output_bytes[i - n_inputs];
    offs[i] = total;
    if (b > kScratchBytes || align_up(b) > kScratchBytes - total)
      return fail(err, PH_ERR_INVALID_ARGUMENT,
                  "ph_dispatch_noalloc: operands need more than the " +
                      std::to_string(kScratchBytes) + "-byte scratch area (operand " +
                      std::to_string(i) + " of " + std::to_string(b) + " bytes ends past it)");
    total += align_up(b);
  }
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return hip_fail(err, e, "hipGetDevice");
  if (device != k->device)
    return fail(err, PH_ERR_INVALID_ARGUMENT,
                "ph_dispatch_noalloc: kernel was loaded on device " + std::to_string(k->device) +
                    ", current device is " + std::to_string(device));
  void *base = nullptr;
  rc = scratch_address(device, &base, err);
  if (rc != PH_OK) return rc;
  char *sbase = static_cast<char *>(base);
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::mutex> in_use(g_scratch_use[device]);
  // Once work is queued, every exit waits for it: a queued copy must not
  // touch the caller's host buffers after we return.
  auto drain_and = [&](int code) {
    (void)hipStreamSynchronize(s);  // best effort: `code` is the error reported
    return code;
  };
  for (size_t i = 0; i < n_inputs; ++i) {
    if (!input_bytes[i]) continue;
    e = hipMemcpyHtoDAsync(sbase + offs[i], const_cast<void *>(inputs[i]), input_bytes[i], s);
    if (e != hipSuccess) return drain_and(hip_fail(err, e, "hipMemcpyHtoDAsync"));
  }
  // Output slots start at zero (the area keeps the previous call's data).
  if (n_outputs) {
    size_t lo = offs[n_inputs];
    size_t words = (total - lo) / 4;
    unsigned int zb = (unsigned int)std::min<size_t>((words + 255) / 256, 2048);
    if (words) {
      hipLaunchKernelGGL(zero_words, dim3(zb), dim3(256), 0, s,
                         reinterpret_cast<uint32_t *>(sbase + lo), words);
      e = hipGetLastError();
      if (e != hipSuccess) return drain_and(hip_fail(err, e, "zero_words launch"));
    }
  }
  void *ptrs[kMaxOperands];
  void *params[kMaxOperands];
  for (size_t i = 0; i < n_ops; ++i) {
    ptrs[i] = sbase + offs[i];
    params[i] = &ptrs[i];
  }
  e = hipModuleLaunchKernel(k->function, blocks, 1, 1, block, 1, 1, 0, s,
                            n_ops ? params : nullptr, nullptr);
  if (e != hipSuccess) return drain_and(hip_fail(err, e, "hipModuleLaunchKernel"));
  for (size_t i = 0; i < n_outputs; ++i) {
    if (!output_bytes[i]) continue;
    e = hipMemcpyDtoHAsync(outputs[i], sbase + offs[n_inputs + i], output_bytes[i], s);
    if (e != hipSuccess) return drain_and(hip_fail(err, e, "hipMemcpyDtoHAsync"));
  }
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
  return PH_OK;
}

int ph_device_count(int *count) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return PH_OK;
}

int ph_device_name(char *buf, size_t len) {
  hipDeviceProp_t prop;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return PH_ERR_RUNTIME;
  // Some drivers leave the marketing name empty: fall back to the arch.
  std::snprintf(buf, len, "%s (%s)", prop.name[0] ? prop.name : "AMD GPU", prop.gcnArchName);
  return PH_OK;
}

int ph_malloc(size_t bytes, void **ptr, char **err) {
  hipError_t e = hipMalloc(ptr, bytes ? bytes : 4);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipMalloc");
}

int ph_free(void *ptr) { return hipFree(ptr) == hipSuccess ? PH_OK : PH_ERR_RUNTIME; }

int ph_host_alloc(size_t bytes, void **ptr, char **err) {
  hipError_t e = hipHostMalloc(ptr, bytes ? bytes : 4, hipHostMallocDefault);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipHostMalloc");
}

int ph_host_free(void *ptr) { return hipHostFree(ptr) == hipSuccess ? PH_OK : PH_ERR_RUNTIME; }

int ph_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream, char **err) {
  hipError_t e = hipMemcpyHtoDAsync(dst, const_cast<void *>(src), bytes, (hipStream_t)stream);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipMemcpyHtoDAsync");
}

int ph_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream, char **err) {
  hipError_t e = hipMemcpyDtoHAsync(dst, const_cast<void *>(src), bytes, (hipStream_t)stream);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipMemcpyDtoHAsync");
}

namespace {

// The pinned buffer small readbacks of ph_memcpy_d2h_wait bounce through:
// one per thread while it lives, returned to a pool at thread exit (no
// HIP call there) for the next thread.
constexpr size_t kReadbackBounce = 64 * 1024;

struct BouncePool {
  std::mutex mutex;
  std::vector<void *> idle;
  static BouncePool &instance() {
    static BouncePool *pool = new BouncePool();  // never destroyed
    return *pool;
  }
};

struct ThreadBounce {
  void *buf = nullptr;
  ~ThreadBounce() {
    if (!buf) return;
    BouncePool &pool = BouncePool::instance();
    std::lock_guard<std::mutex> lock(pool.mutex);
    pool.idle.push_back(buf);
  }
};

int readback_bounce(void **out, char **err) {
  thread_local ThreadBounce mine;
  if (!mine.buf) {
    BouncePool &pool = BouncePool::instance();
    {
      std::lock_guard<std::mutex> lock(pool.mutex);
      if (!pool.idle.empty()) {
        mine.buf = pool.idle.back();
        pool.idle.pop_back();
      }
    }
    if (!mine.buf) {
      hipError_t e = hipHostMalloc(&mine.buf, kReadbackBounce, hipHostMallocDefault);
      if (e != hipSuccess) {
        mine.buf = nullptr;
        return hip_fail(err, e, "hipHostMalloc");
      }
    }
  }
  *out = mine.buf;
  return PH_OK;
}

}  // namespace

int ph_memcpy_d2h_wait(void *dst, const void *src, size_t bytes, void *stream, char **err) {
  // Small readbacks bounce through a per-thread pinned buffer: a DMA into
  // pinned memory plus a memcpy takes about 13 us on MI355X, a copy into
  // pageable memory about 23 us.
  hipStream_t s = (hipStream_t)stream;
  if (bytes <= kReadbackBounce) {
    void *bounce = nullptr;
    int rc = readback_bounce(&bounce, err);
    if (rc != PH_OK) return rc;
    hipError_t e = hipMemcpyDtoHAsync(bounce, const_cast<void *>(src), bytes, s);
    if (e != hipSuccess) return hip_fail(err, e, "hipMemcpyDtoHAsync");
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
    std::memcpy(dst, bounce, bytes);
    return PH_OK;
  }
  hipError_t e = hipMemcpyDtoHAsync(dst, const_cast<void *>(src), bytes, s);
  if (e != hipSuccess) return hip_fail(err, e, "hipMemcpyDtoHAsync");
  e = hipStreamSynchronize(s);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipStreamSynchronize");
}

int ph_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream, char **err) {
  hipError_t e = hipMemcpyDtoDAsync(dst, const_cast<void *>(src), bytes, (hipStream_t)stream);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipMemcpyDtoDAsync");
}

int ph_stream_create(void **stream, char **err) {
  hipStream_t s;
  hipError_t e = hipStreamCreate(&s);
  if (e != hipSuccess) return hip_fail(err, e, "hipStreamCreate");
  *stream = s;
  return PH_OK;
}

int ph_stream_destroy(void *stream) {
  return hipStreamDestroy((hipStream_t)stream) == hipSuccess ? PH_OK : PH_ERR_RUNTIME;
}

int ph_stream_synchronize(void *stream, char **err) {
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipStreamSynchronize");
}

int ph_event_create(void **event, char **err) {
  hipEvent_t ev;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return hip_fail(err, e, "hipEventCreate");
  *event = ev;
  return PH_OK;
}

int ph_event_destroy(void *event) {
  return hipEventDestroy((hipEvent_t)event) == hipSuccess ? PH_OK : PH_ERR_RUNTIME;
}

int ph_event_record(void *event, void *stream, char **err) {
  hipError_t e = hipEventRecord((hipEvent_t)event, (hipStream_t)stream);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipEventRecord");
}

int ph_event_synchronize(void *event, char **err) {
  hipError_t e = hipEventSynchronize((hipEvent_t)event);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipEventSynchronize");
}

int ph_event_query(void *event) {
  hipError_t e = hipEventQuery((hipEvent_t)event);
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  return -1;
}

int ph_event_elapsed_ms(void *start, void *stop, float *ms, char **err) {
  hipError_t e = hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipEventElapsedTime");
}

int ph_device_synchronize(char **err) {
  hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipDeviceSynchronize");
}

int ph_stream_begin_capture(void *stream, char **err) {
  hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipStreamBeginCapture");
}

int ph_stream_end_capture(void *stream, void **graph_exec, char **err) {
  hipGraph_t graph;
  hipError_t e = hipStreamEndCapture((hipStream_t)stream, &graph);
  if (e != hipSuccess) return hip_fail(err, e, "hipStreamEndCapture");
  hipGraphExec_t exec;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);  // the executable graph no longer needs it
  if (e != hipSuccess) return hip_fail(err, e, "hipGraphInstantiate");
  *graph_exec = exec;
  return PH_OK;
}

int ph_graph_launch(void *graph_exec, void *stream, char **err) {
  hipError_t e = hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream);
  return e == hipSuccess ? PH_OK : hip_fail(err, e, "hipGraphLaunch");
}

int ph_graph_destroy(void *graph_exec) {
  return hipGraphExecDestroy((hipGraphExec_t)graph_exec) == hipSuccess ? PH_OK : PH_ERR_RUNTIME;
}

}  // extern "C"
