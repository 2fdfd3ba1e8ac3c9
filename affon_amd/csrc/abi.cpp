// C ABI of the rocm quantized-linear backend: sessions, device memory,
// validation, implementation selection and the host-pointer drop-in.
//
// Validation mirrors the reference exactly:
//   src/js/compute/program.ts:481-494      (operand dtypes, bits, group, shapes)
//   src/support/compute_core_cyna.zig:1000-1022 (overflow-checked counts)
// and rejects before any device work, leaving the output untouched.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>
#include <unordered_set>
#include <vector>

#include "affon_rocm.h"
#include "internal.h"

struct affon_rocm_session {
  int device = 0;
  hipStream_t stream = nullptr;
  affon::Workspace* workspace = nullptr;
  // Allocations made through affon_rocm_alloc and not yet freed: the
  // session frees them when it ends, so tensors that outlive it leak nothing.
  // alloc and free may come from any thread (a caller's garbage collector
  // frees from whichever thread it runs on): the mutex guards the set.
  std::mutex allocations_mutex;
  std::unordered_set<void*> allocations;
};

namespace affon {

Workspace::~Workspace() {
  if (hipSetDevice(device_) != hipSuccess) return;
  if (ptr_ != nullptr) (void)hipFree(ptr_);
  for (void* p : retired_) (void)hipFree(p);
}

void* Workspace::get(size_t bytes) {
  if (bytes <= bytes_) return ptr_;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream_, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone) return nullptr;
  // The old buffer stays allocated (retired) until the session ends: work
  // already enqueued, and graphs captured with its address, may still use it.
  if (ptr_ != nullptr) {
    retired_.push_back(ptr_);
    retired_bytes_ = bytes_;
  }
  ptr_ = nullptr;
  bytes_ = 0;
  // Grow at least twofold, so that retired buffers stay few.
  const size_t want = bytes > 2 * retired_bytes_ ? bytes : 2 * retired_bytes_;
  const size_t rounded = (want + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
  if (hipMalloc(&ptr_, rounded) != hipSuccess) {
    ptr_ = nullptr;
    (void)hipGetLastError();
    return nullptr;
  }
  if (hipMemset(ptr_, 0, rounded) != hipSuccess) {
    (void)hipFree(ptr_);
    ptr_ = nullptr;
    (void)hipGetLastError();
    return nullptr;
  }
  bytes_ = rounded;
  return ptr_;
}

}  // namespace affon

// Scratch memory of affon_rocm_quantized_matmul_noalloc: the split-K partial
// sums of the tiled kernels and the reassociated prefill GEMM's per-group
// activation sums, in a static device array (one per GPU, held until the
// process ends): 32 MiB of partial sums (four K ranges of a 512 x 4096 f32
// output) plus 1 MiB of group sums. Host code uses only the per-device
// address that hipGetSymbolAddress returns for it (kept by scratch_on), never
// the array's name, which on the host is a stand-in and not a device address.
constexpr size_t kNoAllocScratchBytes = (size_t(32) << 20) + (size_t(1) << 20);
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

// Device address of `scratch` on `device`, looked up on the first
// no-allocation call on that device, with the device current (check_session
// has made it so); only a successful lookup is kept, so a failed one is
// retried by the next call.
std::mutex g_scratch_mutex;
void* g_scratch_ptr[64] = {};

hipError_t scratch_on(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

thread_local std::string g_last_error;

int fail(int status, const char* format, ...) {
  char buffer[512];
  va_list args;
  va_start(args, format);
  std::vsnprintf(buffer, sizeof(buffer), format, args);
  va_end(args);
  g_last_error = buffer;
  return status;
}

int hip_fail(hipError_t error, const char* what) {
  return fail(AFFON_ROCM_HIP_ERROR, "%s: %s", what, hipGetErrorString(error));
}

void clear_error() { g_last_error.clear(); }

bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
  *out = a * b;
  return true;
}

bool add_ok(uint64_t a, uint64_t b, uint64_t* out) {
  if (b > std::numeric_limits<uint64_t>::max() - a) return false;
  *out = a + b;
  return true;
}

int element_size(int dtype) {
  switch (dtype) {
    case AFFON_ROCM_F32: return 4;
    case AFFON_ROCM_BF16: return 2;
    case AFFON_ROCM_U32: return 4;
    default: return 0;
  }
}

bool is_float_dtype(int dtype) { return dtype == AFFON_ROCM_F32 || dtype == AFFON_ROCM_BF16; }

// Checks that every element a view names lies inside its allocation.
int check_view(const affon_rocm_view& v, const char* name) {
  const int esize = element_size(v.dtype);
  if (v.data == nullptr) return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul %s has no data", name);
  if (v.shape[0] <= 0 || v.shape[1] <= 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul %s has an empty dimension", name);
  if (v.stride[0] < 0 || v.stride[1] < 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul %s has a negative stride", name);
  if (v.byte_offset % static_cast<size_t>(esize) != 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul %s byte offset is not element aligned", name);
  uint64_t last0 = 0, last1 = 0, last = 0, bytes = 0, end = 0;
  if (!mul_ok(static_cast<uint64_t>(v.shape[0] - 1), static_cast<uint64_t>(v.stride[0]), &last0) ||
      !mul_ok(static_cast<uint64_t>(v.shape[1] - 1), static_cast<uint64_t>(v.stride[1]), &last1) ||
      !add_ok(last0, last1, &last) || !add_ok(last, 1, &last) ||
      !mul_ok(last, static_cast<uint64_t>(esize), &bytes) ||
      !add_ok(bytes, static_cast<uint64_t>(v.byte_offset), &end))
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul %s extent overflows", name);
  if (end > v.buffer_bytes)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul %s view exceeds its buffer (%llu > %llu bytes)", name,
                static_cast<unsigned long long>(end), static_cast<unsigned long long>(v.buffer_bytes));
  return AFFON_ROCM_OK;
}

// program.ts:483-493 and compute_core_cyna.zig:1012-1022.
int validate(const affon_rocm_qmm_desc* d, affon::QmmProblem* p) {
  if (d == nullptr) return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul descriptor is null");
  if (d->bits != 2 && d->bits != 4 && d->bits != 8)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul bits must be 2, 4, or 8");
  if (d->group_size == 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul group_size must be a positive integer");
  if (!is_float_dtype(d->input.dtype) || d->packed.dtype != AFFON_ROCM_U32 || !is_float_dtype(d->scales.dtype) ||
      d->biases.dtype != d->scales.dtype)
    return fail(AFFON_ROCM_INVALID_SHAPE,
                "quantized_matmul requires f32/bf16 input, u32 weights, and matching f32/bf16 scales and biases");
  const int64_t M = d->input.shape[0], K = d->input.shape[1], N = d->packed.shape[0];
  const int64_t per_word = 32 / static_cast<int64_t>(d->bits);
  const int64_t g = static_cast<int64_t>(d->group_size);
  if (M <= 0 || K <= 0 || N <= 0 || K % per_word != 0 || K % g != 0 || d->packed.shape[1] != K / per_word ||
      d->scales.shape[0] != N || d->scales.shape[1] != K / g || d->biases.shape[0] != N ||
      d->biases.shape[1] != K / g)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul packed or group dimensions do not match input features");
  int status;
  if ((status = check_view(d->input, "input")) != AFFON_ROCM_OK) return status;
  if ((status = check_view(d->packed, "packed")) != AFFON_ROCM_OK) return status;
  if ((status = check_view(d->scales, "scales")) != AFFON_ROCM_OK) return status;
  if ((status = check_view(d->biases, "biases")) != AFFON_ROCM_OK) return status;
  uint64_t out_count = 0, out_bytes = 0;
  if (!mul_ok(static_cast<uint64_t>(M), static_cast<uint64_t>(N), &out_count) || !mul_ok(out_count, 4, &out_bytes))
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul output size overflows");
  if (d->output == nullptr || d->output_bytes < out_bytes)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul output buffer is smaller than [M,N] f32");
  if (d->implementation < AFFON_ROCM_IMPL_AUTO || d->implementation > AFFON_ROCM_IMPL_MFMA)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul unknown implementation %d", d->implementation);
  if (d->numerical_policy < AFFON_ROCM_BACKEND_EQUIVALENT || d->numerical_policy > AFFON_ROCM_APPROXIMATE)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul unknown numerical policy %d", d->numerical_policy);

  p->M = M;
  p->N = N;
  p->K = K;
  p->bits = static_cast<int>(d->bits);
  p->group = g;
  p->x = static_cast<const uint8_t*>(d->input.data) + d->input.byte_offset;
  p->xs0 = d->input.stride[0];
  p->xs1 = d->input.stride[1];
  p->x_dtype = d->input.dtype;
  p->w = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(d->packed.data) + d->packed.byte_offset);
  p->ws0 = d->packed.stride[0];
  p->ws1 = d->packed.stride[1];
  p->s = static_cast<const uint8_t*>(d->scales.data) + d->scales.byte_offset;
  p->ss0 = d->scales.stride[0];
  p->ss1 = d->scales.stride[1];
  p->b = static_cast<const uint8_t*>(d->biases.data) + d->biases.byte_offset;
  p->bs0 = d->biases.stride[0];
  p->bs1 = d->biases.stride[1];
  p->p_dtype = d->scales.dtype;
  p->out = d->output;
  return AFFON_ROCM_OK;
}

// Registered candidates, in the order AUTO prefers them.
struct Candidate {
  int impl;
  const char* id;
  int version;
  // 0 exact (bit-identical to the ordered CPU loop), 1 reassociated,
  // 2 approximate (rounds decoded weights to bf16).
  int numerical_class;
  bool (*supports)(const affon::QmmProblem&);
  hipError_t (*launch)(const affon::QmmProblem&, const affon::Launch&);
};

const Candidate kCandidates[] = {
    {AFFON_ROCM_IMPL_MFMA, "rocm_quantized_matmul.mfma", 1, 2, affon::mfma_supports, affon::mfma_launch},
    {AFFON_ROCM_IMPL_GEMV_MFMA, "rocm_quantized_matmul.gemv_mfma", 1, 1, affon::gemv_mfma_supports,
     affon::gemv_mfma_launch},
    {AFFON_ROCM_IMPL_GEMV, "rocm_quantized_matmul.gemv", 1, 1, affon::gemv_supports, affon::gemv_launch},
    {AFFON_ROCM_IMPL_GENERIC, "rocm_quantized_matmul.generic", 1, 0, affon::generic_supports,
     affon::generic_launch},
};

bool policy_accepts(int policy, int numerical_class) {
  switch (policy) {
    case AFFON_ROCM_EXACT_ONLY: return numerical_class == 0;
    case AFFON_ROCM_BACKEND_EQUIVALENT: return numerical_class <= 1;
    default: return true;
  }
}

// Shape rule for AUTO among candidates that pass their guards: the prefill
// GEMM for M >= 64 (when the policy admits its approximate class), the MFMA
// decode kernels for M >= 2 with bf16 input (the reassociated class's path
// for prefill: from 128 rows the large-tile reassociated GEMM, gemm_re.hip,
// where it takes the shape, else row tiles of 32), the VALU decode kernel
// otherwise, the generic kernel last.
bool auto_prefers(const Candidate& c, const affon::QmmProblem& p) {
  switch (c.impl) {
    case AFFON_ROCM_IMPL_MFMA: return p.M >= 64;
    case AFFON_ROCM_IMPL_GEMV_MFMA: return p.M >= 2;
    default: return true;
  }
}

int select(const affon_rocm_qmm_desc* d, const affon::QmmProblem& p, const Candidate** out) {
  for (const Candidate& c : kCandidates) {
    if (d->implementation != AFFON_ROCM_IMPL_AUTO && d->implementation != c.impl) continue;
    if (!policy_accepts(d->numerical_policy, c.numerical_class)) {
      if (d->implementation == c.impl)
        return fail(AFFON_ROCM_UNSUPPORTED, "%s is not allowed under the requested numerical policy", c.id);
      continue;
    }
    if (!c.supports(p)) {
      if (d->implementation == c.impl)
        return fail(AFFON_ROCM_UNSUPPORTED, "%s cannot run this shape or layout", c.id);
      continue;
    }
    if (d->implementation == AFFON_ROCM_IMPL_AUTO && !auto_prefers(c, p)) continue;
    *out = &c;
    return AFFON_ROCM_OK;
  }
  return fail(AFFON_ROCM_UNSUPPORTED, "no quantized_matmul implementation accepts this problem");
}

int check_session(affon_rocm_session* s) {
  if (s == nullptr || s->stream == nullptr) return fail(AFFON_ROCM_CORE_FAILURE, "session is not open");
  hipError_t e = hipSetDevice(s->device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  return AFFON_ROCM_OK;
}

bool is_gfx950(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return false;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

}  // namespace

extern "C" {

int affon_rocm_device_count(int* count) {
  clear_error();
  if (count == nullptr) return fail(AFFON_ROCM_CORE_FAILURE, "count is null");
  *count = 0;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) return AFFON_ROCM_OK;
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  for (int i = 0; i < n; ++i) *count += is_gfx950(i) ? 1 : 0;
  return AFFON_ROCM_OK;
}

int affon_rocm_session_create(int device, affon_rocm_session** out) {
  clear_error();
  if (out == nullptr) return fail(AFFON_ROCM_CORE_FAILURE, "session output is null");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || device < 0 || device >= n)
    return fail(AFFON_ROCM_UNSUPPORTED, "rocm backend unavailable: no HIP device %d", device);
  if (!is_gfx950(device)) return fail(AFFON_ROCM_UNSUPPORTED, "rocm backend unavailable: device %d is not gfx950", device);
  if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
  hipStream_t stream = nullptr;
  if ((e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking)) != hipSuccess) return hip_fail(e, "hipStreamCreate");
  auto* session = new affon_rocm_session;
  session->device = device;
  session->stream = stream;
  session->workspace = new affon::Workspace(device, stream);
  *out = session;
  return AFFON_ROCM_OK;
}

int affon_rocm_session_destroy(affon_rocm_session* session) {
  clear_error();
  if (session == nullptr) return AFFON_ROCM_OK;
  int status = AFFON_ROCM_OK;
  if (hipSetDevice(session->device) == hipSuccess && session->stream != nullptr) {
    hipError_t e = hipStreamSynchronize(session->stream);
    if (e != hipSuccess) status = hip_fail(e, "hipStreamSynchronize");
    {
      std::lock_guard<std::mutex> lock(session->allocations_mutex);
      for (void* ptr : session->allocations) (void)hipFree(ptr);
      session->allocations.clear();
    }
    delete session->workspace;
    e = hipStreamDestroy(session->stream);
    if (e != hipSuccess && status == AFFON_ROCM_OK) status = hip_fail(e, "hipStreamDestroy");
  } else {
    delete session->workspace;
  }
  delete session;
  return status;
}

void* affon_rocm_session_stream(affon_rocm_session* session) {
  return session == nullptr ? nullptr : static_cast<void*>(session->stream);
}

int affon_rocm_alloc(affon_rocm_session* session, size_t bytes, void** out) {
  clear_error();
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  if (out == nullptr) return fail(AFFON_ROCM_CORE_FAILURE, "allocation output is null");
  *out = nullptr;
  hipError_t e = hipMalloc(out, bytes == 0 ? 1 : bytes);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  std::lock_guard<std::mutex> lock(session->allocations_mutex);
  session->allocations.insert(*out);
  return AFFON_ROCM_OK;
}

int affon_rocm_free(affon_rocm_session* session, void* ptr) {
  clear_error();
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  if (ptr == nullptr) return AFFON_ROCM_OK;
  {
    std::lock_guard<std::mutex> lock(session->allocations_mutex);
    if (session->allocations.erase(ptr) == 0)
      return fail(AFFON_ROCM_CORE_FAILURE, "free of memory this session did not allocate");
  }
  hipError_t e = hipStreamSynchronize(session->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  e = hipFree(ptr);
  if (e != hipSuccess) return hip_fail(e, "hipFree");
  return AFFON_ROCM_OK;
}

static int copy(affon_rocm_session* session, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  clear_error();
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  if (bytes == 0) return AFFON_ROCM_OK;
  if (dst == nullptr || src == nullptr) return fail(AFFON_ROCM_CORE_FAILURE, "copy with a null pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, session->stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
  e = hipStreamSynchronize(session->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  return AFFON_ROCM_OK;
}

int affon_rocm_memcpy_h2d(affon_rocm_session* session, void* dst, const void* src, size_t bytes) {
  return copy(session, dst, src, bytes, hipMemcpyHostToDevice);
}

int affon_rocm_memcpy_d2h(affon_rocm_session* session, void* dst, const void* src, size_t bytes) {
  return copy(session, dst, src, bytes, hipMemcpyDeviceToHost);
}

int affon_rocm_memcpy_d2d(affon_rocm_session* session, void* dst, const void* src, size_t bytes) {
  return copy(session, dst, src, bytes, hipMemcpyDeviceToDevice);
}

int affon_rocm_synchronize(affon_rocm_session* session) {
  clear_error();
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  hipError_t e = hipStreamSynchronize(session->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  return AFFON_ROCM_OK;
}

const char* affon_rocm_last_error(void) { return g_last_error.c_str(); }

int affon_rocm_quantized_matmul(affon_rocm_session* session, const affon_rocm_qmm_desc* desc) {
  clear_error();
  affon::QmmProblem p;
  int status = validate(desc, &p);
  if (status != AFFON_ROCM_OK) return status;
  const Candidate* c = nullptr;
  if ((status = select(desc, p, &c)) != AFFON_ROCM_OK) return status;
  if ((status = check_session(session)) != AFFON_ROCM_OK) return status;
  affon::Launch launch;
  launch.stream = session->stream;
  launch.workspace = session->workspace;
  hipError_t e = c->launch(p, launch);
  if (e != hipSuccess) return hip_fail(e, c->id);
  return AFFON_ROCM_OK;
}

int affon_rocm_quantized_matmul_noalloc(affon_rocm_session* session, const affon_rocm_qmm_desc* desc) {
  clear_error();
  affon::QmmProblem p;
  int status = validate(desc, &p);
  if (status != AFFON_ROCM_OK) return status;
  const Candidate* c = nullptr;
  if ((status = select(desc, p, &c)) != AFFON_ROCM_OK) return status;
  if ((status = check_session(session)) != AFFON_ROCM_OK) return status;
  void* fixed = nullptr;
  if (hipError_t e = scratch_on(session->device, &fixed); e != hipSuccess)
    return hip_fail(e, "hipGetSymbolAddress(scratch)");
  affon::Launch launch;
  launch.stream = session->stream;
  launch.fixed = fixed;
  launch.fixed_bytes = kNoAllocScratchBytes;
  hipError_t e = c->launch(p, launch);
  if (launch.fixed_short > 0)
    return fail(AFFON_ROCM_UNSUPPORTED,
                "%s needs %zu bytes of split-K scratch for this shape, more than the %zu bytes the no-allocation "
                "entry point holds; use affon_rocm_quantized_matmul",
                c->id, launch.fixed_short, kNoAllocScratchBytes);
  if (e != hipSuccess) return hip_fail(e, c->id);
  return AFFON_ROCM_OK;
}

int affon_rocm_read_floor(affon_rocm_session* session, const void* const* buffers, const uint64_t* bytes, int count,
                          void* sink) {
  clear_error();
  if (buffers == nullptr || bytes == nullptr || sink == nullptr || count < 1 || count > 4)
    return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor needs 1 to 4 buffers, their sizes and a sink word");
  for (int i = 0; i < count; ++i) {
    if (buffers[i] == nullptr || reinterpret_cast<uintptr_t>(buffers[i]) % 16 != 0 || bytes[i] < 16)
      return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor buffer %d is null, unaligned or shorter than 16 bytes", i);
  }
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  hipError_t e = affon::read_floor_launch(buffers, bytes, count, static_cast<uint32_t*>(sink), session->stream);
  if (e != hipSuccess) return hip_fail(e, "read_floor");
  return AFFON_ROCM_OK;
}

int affon_rocm_read_floor_geometry(affon_rocm_session* session, const void* buffer, uint64_t bytes, void* sink,
                                   uint64_t sink_bytes, const affon_rocm_floor_geometry* geometry) {
  clear_error();
  if (geometry == nullptr || buffer == nullptr || sink == nullptr)
    return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor_geometry needs a buffer, a sink and a geometry");
  const affon_rocm_floor_geometry g = *geometry;
  if (reinterpret_cast<uintptr_t>(buffer) % 16 != 0 || reinterpret_cast<uintptr_t>(sink) % 8 != 0 || bytes < 16 ||
      bytes % 16 != 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor_geometry: buffer unaligned, or bytes not a positive multiple of 16");
  if (g.kib_per_wave != 1 && g.kib_per_wave != 2 && g.kib_per_wave != 4 && g.kib_per_wave != 8)
    return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor_geometry: kib_per_wave must be 1, 2, 4 or 8");
  if (g.threads < 64 || g.threads > 1024 || g.threads % 64 != 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor_geometry: threads must be a multiple of 64 from 64 to 1024");
  if (g.valu_per_wave < 0 || g.valu_per_wave > 4096 || g.valu_per_wave % 8 != 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor_geometry: valu_per_wave must be a multiple of 8 from 0 to 4096");
  if (g.store_every < 0) return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor_geometry: store_every must be >= 0");
  const uint64_t waves = affon::read_geometry_waves(bytes, g.kib_per_wave);
  const uint64_t need = g.store_every > 0 ? 8 * ((waves + g.store_every - 1) / g.store_every) : 4;
  if (sink_bytes < need)
    return fail(AFFON_ROCM_INVALID_SHAPE, "read_floor_geometry: sink holds %llu bytes, the stores need %llu",
                static_cast<unsigned long long>(sink_bytes), static_cast<unsigned long long>(need));
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  hipError_t e = affon::read_geometry_launch(buffer, bytes, static_cast<float*>(sink), g.kib_per_wave, g.threads,
                                             g.store_every, g.valu_per_wave, session->stream);
  if (e != hipSuccess) return hip_fail(e, "read_floor_geometry");
  return AFFON_ROCM_OK;
}

int affon_rocm_empty_launch(affon_rocm_session* session, uint32_t blocks, uint32_t threads) {
  clear_error();
  if (blocks < 1 || blocks > 0x7fffffffu || threads < 1 || threads > 1024)
    return fail(AFFON_ROCM_INVALID_SHAPE, "empty_launch: 1 to 2^31-1 workgroups of 1 to 1024 threads");
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  hipError_t e = affon::empty_launch(blocks, threads, session->stream);
  if (e != hipSuccess) return hip_fail(e, "empty_launch");
  return AFFON_ROCM_OK;
}

int affon_rocm_kernel_supports(const affon_rocm_qmm_desc* desc, const char* kernel, int* supported) {
  clear_error();
  if (kernel == nullptr || supported == nullptr)
    return fail(AFFON_ROCM_INVALID_SHAPE, "kernel_supports needs a kernel name and a result pointer");
  affon::QmmProblem p;
  int status = validate(desc, &p);
  if (status != AFFON_ROCM_OK) return status;
  static const struct {
    const char* name;
    bool (*guard)(const affon::QmmProblem&);
  } kGuards[] = {
      {"generic", affon::generic_supports}, {"gemv", affon::gemv_supports},     {"gemv1", affon::gemv1_supports},
      {"gemv_mfma", affon::gemv_mfma_supports}, {"mfma", affon::mfma_supports}, {"gemm_re", affon::re_gemm_supports},
      {"gemm_pair", affon::pair_supports},  {"gemm_re32", affon::re32_supports},
  };
  for (const auto& g : kGuards) {
    if (std::strcmp(g.name, kernel) == 0) {
      *supported = g.guard(p) ? 1 : 0;
      return AFFON_ROCM_OK;
    }
  }
  return fail(AFFON_ROCM_INVALID_SHAPE, "kernel_supports: unknown kernel '%s'", kernel);
}

int affon_rocm_quantized_matmul_select(const affon_rocm_qmm_desc* desc, char* id, size_t cap) {
  clear_error();
  affon::QmmProblem p;
  int status = validate(desc, &p);
  if (status != AFFON_ROCM_OK) return status;
  const Candidate* c = nullptr;
  if ((status = select(desc, p, &c)) != AFFON_ROCM_OK) return status;
  if (id != nullptr && cap > 0) {
    std::strncpy(id, c->id, cap - 1);
    id[cap - 1] = '\0';
  }
  return AFFON_ROCM_OK;
}

}  // extern "C"

namespace {

// How a fused call runs: the first problem (the only one, or the gate
// projection), and for a two-launch SiLU gate the up projection, whose
// kernel multiplies silu(stored gate) into its output.
struct FusedPlan {
  affon::QmmProblem first, second;
  const Candidate* first_c = nullptr;
  const Candidate* second_c = nullptr;
  bool two = false;
};

bool same_layout(const affon_rocm_view& a, const affon_rocm_view& b) {
  return a.stride[0] == b.stride[0] && a.stride[1] == b.stride[1];
}

int plan_fused(const affon_rocm_qmm_desc* d, const affon_rocm_qmm_epilogue* e, FusedPlan* plan) {
  if (e == nullptr) return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul epilogue is null");
  int status = validate(d, &plan->first);
  if (status != AFFON_ROCM_OK) return status;
  affon::QmmProblem& p = plan->first;
  switch (e->kind) {
    case AFFON_ROCM_EPILOGUE_NONE:
      return select(d, p, &plan->first_c);
    case AFFON_ROCM_EPILOGUE_BIAS: {
      const int esize = element_size(e->bias_dtype);
      if (e->bias == nullptr || !is_float_dtype(e->bias_dtype))
        return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul output bias must be an f32/bf16 vector");
      if (e->bias_bytes / static_cast<size_t>(esize) < static_cast<size_t>(p.N) ||
          reinterpret_cast<uintptr_t>(e->bias) % static_cast<uintptr_t>(esize) != 0)
        return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul output bias needs N aligned elements");
      p.epi.kind = affon::kEpiBias;
      p.epi.bias = static_cast<const uint8_t*>(e->bias);
      p.epi.bias_bf16 = e->bias_dtype == AFFON_ROCM_BF16;
      return select(d, p, &plan->first_c);
    }
    case AFFON_ROCM_EPILOGUE_SILU_GATE: {
      const affon_rocm_view* gate[3] = {&d->packed, &d->scales, &d->biases};
      const affon_rocm_view* up[3] = {&e->up_packed, &e->up_scales, &e->up_biases};
      const char* names[3] = {"up packed", "up scales", "up biases"};
      for (int i = 0; i < 3; ++i) {
        if (up[i]->dtype != gate[i]->dtype || up[i]->shape[0] != gate[i]->shape[0] ||
            up[i]->shape[1] != gate[i]->shape[1])
          return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul %s must match the gate projection's shape and dtype",
                      names[i]);
        if ((status = check_view(*up[i], names[i])) != AFFON_ROCM_OK) return status;
      }
      affon::QmmProblem& q = plan->second;
      q = p;
      q.w = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(e->up_packed.data) +
                                              e->up_packed.byte_offset);
      q.ws0 = e->up_packed.stride[0];
      q.ws1 = e->up_packed.stride[1];
      q.s = static_cast<const uint8_t*>(e->up_scales.data) + e->up_scales.byte_offset;
      q.ss0 = e->up_scales.stride[0];
      q.ss1 = e->up_scales.stride[1];
      q.b = static_cast<const uint8_t*>(e->up_biases.data) + e->up_biases.byte_offset;
      q.bs0 = e->up_biases.stride[0];
      q.bs1 = e->up_biases.stride[1];
      if ((status = select(d, p, &plan->first_c)) != AFFON_ROCM_OK) return status;
      // One launch when the gate's kernel pairs rows of both projections.
      affon::QmmProblem paired = p;
      paired.epi.kind = affon::kEpiSiluPair;
      paired.epi.w2 = q.w;
      paired.epi.s2 = q.s;
      paired.epi.b2 = q.b;
      if (plan->first_c->impl == AFFON_ROCM_IMPL_GEMV && same_layout(d->packed, e->up_packed) &&
          same_layout(d->scales, e->up_scales) && same_layout(d->biases, e->up_biases) &&
          affon::gemv_pair_supports(paired)) {
        p = paired;
        return AFFON_ROCM_OK;
      }
      plan->two = true;
      q.epi.kind = affon::kEpiGateMul;
      return select(d, q, &plan->second_c);
    }
    default:
      return fail(AFFON_ROCM_INVALID_SHAPE, "quantized_matmul unknown epilogue %d", e->kind);
  }
}

std::string fused_text(const FusedPlan& plan);
int copy_id(const std::string& text, char* id, size_t cap);

}  // namespace

extern "C" {

int affon_rocm_quantized_matmul_fused(affon_rocm_session* session, const affon_rocm_qmm_desc* desc,
                                      const affon_rocm_qmm_epilogue* epilogue) {
  clear_error();
  FusedPlan plan;
  int status = plan_fused(desc, epilogue, &plan);
  if (status != AFFON_ROCM_OK) return status;
  if ((status = check_session(session)) != AFFON_ROCM_OK) return status;
  affon::Launch launch;
  launch.stream = session->stream;
  launch.workspace = session->workspace;
  hipError_t e = plan.first_c->launch(plan.first, launch);
  if (e != hipSuccess) return hip_fail(e, plan.first_c->id);
  if (plan.two) {
    e = plan.second_c->launch(plan.second, launch);
    if (e != hipSuccess) return hip_fail(e, plan.second_c->id);
  }
  return AFFON_ROCM_OK;
}

int affon_rocm_quantized_matmul_fused_select(const affon_rocm_qmm_desc* desc, const affon_rocm_qmm_epilogue* epilogue,
                                             char* id, size_t cap) {
  clear_error();
  FusedPlan plan;
  int status = plan_fused(desc, epilogue, &plan);
  if (status != AFFON_ROCM_OK) return status;
  return copy_id(fused_text(plan), id, cap);
}

}  // extern "C"

namespace {

bool same_view(const affon_rocm_view& a, const affon_rocm_view& b) {
  return a.data == b.data && a.byte_offset == b.byte_offset && a.shape[0] == b.shape[0] && a.shape[1] == b.shape[1] &&
         a.stride[0] == b.stride[0] && a.stride[1] == b.stride[1] && a.dtype == b.dtype;
}

// A grouped call: every member's plan, and whether they run as one launch.
struct GroupPlan {
  FusedPlan members[affon::kMaxGroup];
  std::vector<FusedPlan> many;  // more members than one launch takes
  size_t count = 0;
  bool one_launch = false;
  int one_impl = 0;  // the candidate whose kernel runs the whole group
  const FusedPlan& at(size_t i) const { return count <= affon::kMaxGroup ? members[i] : many[i]; }
};

int plan_grouped(const affon_rocm_qmm_desc* descs, const affon_rocm_qmm_epilogue* epilogues, size_t count,
                 GroupPlan* plan) {
  if (descs == nullptr || count == 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "grouped quantized_matmul needs at least one descriptor");
  if (count > affon::kMaxGroup) plan->many.resize(count);
  plan->count = count;
  affon_rocm_qmm_epilogue none;
  std::memset(&none, 0, sizeof(none));
  none.kind = AFFON_ROCM_EPILOGUE_NONE;
  for (size_t i = 0; i < count; ++i) {
    const affon_rocm_qmm_desc& d = descs[i];
    if (i > 0 && (!same_view(d.input, descs[0].input) || d.bits != descs[0].bits ||
                  d.group_size != descs[0].group_size || d.implementation != descs[0].implementation ||
                  d.numerical_policy != descs[0].numerical_policy))
      return fail(AFFON_ROCM_INVALID_SHAPE, "grouped quantized_matmul descriptors must share the input and options");
    const affon_rocm_qmm_epilogue* e = epilogues != nullptr ? &epilogues[i] : &none;
    if (e->kind != AFFON_ROCM_EPILOGUE_NONE && e->kind != AFFON_ROCM_EPILOGUE_BIAS)
      return fail(AFFON_ROCM_INVALID_SHAPE, "grouped quantized_matmul takes no epilogue or an output bias per call");
    FusedPlan& member = count <= affon::kMaxGroup ? plan->members[i] : plan->many[i];
    int status = plan_fused(&d, e, &member);
    if (status != AFFON_ROCM_OK) return status;
  }
  if (count >= 2 && count <= affon::kMaxGroup) {
    affon::QmmProblem problems[affon::kMaxGroup];
    const int impl = plan->members[0].first_c->impl;
    bool same = true;
    for (size_t i = 0; i < count; ++i) {
      problems[i] = plan->members[i].first;
      same = same && plan->members[i].first_c->impl == impl;
    }
    const int n = static_cast<int>(count);
    if (same && impl == AFFON_ROCM_IMPL_GEMV)
      plan->one_launch = affon::gemv_group_supports(problems, n);
    else if (same && impl == AFFON_ROCM_IMPL_GEMV_MFMA)
      plan->one_launch = affon::gemv_mfma_group_supports(problems, n);
    plan->one_impl = impl;
  }
  return AFFON_ROCM_OK;
}

std::string fused_text(const FusedPlan& plan) {
  std::string text = plan.first_c->id;
  switch (plan.first.epi.kind) {
    case affon::kEpiBias: text += "[bias]"; break;
    case affon::kEpiSiluPair: text += "[silu_gate]"; break;
    default: break;
  }
  if (plan.two) text += std::string(";") + plan.second_c->id + "[gate_mul]";
  return text;
}

int copy_id(const std::string& text, char* id, size_t cap) {
  if (id != nullptr && cap > 0) {
    std::strncpy(id, text.c_str(), cap - 1);
    id[cap - 1] = '\0';
  }
  return AFFON_ROCM_OK;
}

}  // namespace

extern "C" {

int affon_rocm_quantized_matmul_grouped(affon_rocm_session* session, const affon_rocm_qmm_desc* descs,
                                        const affon_rocm_qmm_epilogue* epilogues, size_t count) {
  clear_error();
  GroupPlan plan;
  int status = plan_grouped(descs, epilogues, count, &plan);
  if (status != AFFON_ROCM_OK) return status;
  if ((status = check_session(session)) != AFFON_ROCM_OK) return status;
  affon::Launch launch;
  launch.stream = session->stream;
  launch.workspace = session->workspace;
  if (plan.one_launch) {
    affon::QmmProblem problems[affon::kMaxGroup];
    for (size_t i = 0; i < count; ++i) problems[i] = plan.members[i].first;
    const int n = static_cast<int>(count);
    hipError_t e = plan.one_impl == AFFON_ROCM_IMPL_GEMV ? affon::gemv_group_launch(problems, n, launch)
                                                         : affon::gemv_mfma_group_launch(problems, n, launch);
    if (e != hipSuccess) return hip_fail(e, "grouped quantized_matmul");
    return AFFON_ROCM_OK;
  }
  for (size_t i = 0; i < count; ++i) {
    const FusedPlan& member = plan.at(i);
    hipError_t e = member.first_c->launch(member.first, launch);
    if (e != hipSuccess) return hip_fail(e, member.first_c->id);
  }
  return AFFON_ROCM_OK;
}

int affon_rocm_quantized_matmul_grouped_select(const affon_rocm_qmm_desc* descs,
                                               const affon_rocm_qmm_epilogue* epilogues, size_t count, char* id,
                                               size_t cap) {
  clear_error();
  GroupPlan plan;
  int status = plan_grouped(descs, epilogues, count, &plan);
  if (status != AFFON_ROCM_OK) return status;
  if (plan.one_launch) {
    bool bias = false;
    for (size_t i = 0; i < count; ++i) bias = bias || plan.members[i].first.epi.kind == affon::kEpiBias;
    return copy_id(std::string(plan.members[0].first_c->id) + "[grouped:" + std::to_string(count) +
                       (bias ? ",bias]" : "]"),
                   id, cap);
  }
  std::string text;
  for (size_t i = 0; i < count; ++i) text += (i ? ";" : "") + fused_text(plan.at(i));
  return copy_id(text, id, cap);
}

const char* affon_rocm_quantized_matmul_capabilities(void) {
  static const char* kJson =
      "["
      "{\"id\":\"rocm_quantized_matmul.mfma\",\"version\":1,\"numerical_class\":\"approximate\","
      "\"guard\":\"gfx950; bf16 input; group_size % 32 == 0; K % 64 == 0; unit inner strides; M >= 64 when auto\","
      "\"note\":\"decoded weights rounded to bf16 in LDS, bf16 MFMA, f32 accumulation\"},"
      "{\"id\":\"rocm_quantized_matmul.gemv_mfma\",\"version\":1,\"numerical_class\":\"reassociated\","
      "\"guard\":\"gfx950; bf16 input; group_size a power of two >= 64; K % 256 == 0; unit inner strides; M >= 2 when auto (rows beyond 32 in row tiles)\","
      "\"note\":\"integer codes exact in bf16, per-group scale and bias applied in f32\"},"
      "{\"id\":\"rocm_quantized_matmul.gemv\",\"version\":1,\"numerical_class\":\"reassociated\","
      "\"guard\":\"gfx950; group_size % (32/bits) == 0; unit inner strides; aligned rows\","
      "\"note\":\"VALU decode, f32 accumulation, per-group scale and bias applied in f32\"},"
      "{\"id\":\"rocm_quantized_matmul.generic\",\"version\":1,\"numerical_class\":\"exact\","
      "\"guard\":\"gfx950; any strides, byte offsets and group sizes\","
      "\"note\":\"ordered f32 loop per output, separately rounded products and sums\"}"
      "]";
  return kJson;
}

int affon_rocm_quantize(affon_rocm_session* session, const void* weights, int32_t weight_dtype, int64_t rows,
                        int64_t columns, uint32_t bits, uint32_t group_size, uint32_t* packed, void* scales,
                        void* biases, int32_t param_dtype) {
  clear_error();
  if (bits != 2 && bits != 4 && bits != 8) return fail(AFFON_ROCM_INVALID_SHAPE, "quantize bits must be 2, 4, or 8");
  if (group_size == 0) return fail(AFFON_ROCM_INVALID_SHAPE, "quantize group_size must be a positive integer");
  if (!is_float_dtype(weight_dtype) || !is_float_dtype(param_dtype))
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantize requires f32/bf16 weights and f32/bf16 parameters");
  const int64_t per_word = 32 / static_cast<int64_t>(bits);
  if (rows <= 0 || columns <= 0 || columns % per_word != 0 || columns % static_cast<int64_t>(group_size) != 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantize columns must divide into complete words and groups");
  uint64_t count = 0;
  if (!mul_ok(static_cast<uint64_t>(rows), static_cast<uint64_t>(columns), &count) || count > (uint64_t(1) << 60))
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantize size overflows");
  if (weights == nullptr || packed == nullptr || scales == nullptr || biases == nullptr)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantize buffer is null");
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  hipError_t e = affon::quantize_launch(weights, weight_dtype, rows, columns, static_cast<int>(bits), group_size,
                                        packed, scales, biases, param_dtype, session->stream);
  if (e != hipSuccess) return hip_fail(e, "quantize");
  return AFFON_ROCM_OK;
}

int affon_rocm_dequantize(affon_rocm_session* session, const uint32_t* packed, const void* scales, const void* biases,
                          int32_t param_dtype, int64_t rows, int64_t columns, uint32_t bits, uint32_t group_size,
                          void* out, int32_t out_dtype) {
  clear_error();
  if (bits != 2 && bits != 4 && bits != 8)
    return fail(AFFON_ROCM_INVALID_SHAPE, "dequantize bits must be 2, 4, or 8");
  if (group_size == 0) return fail(AFFON_ROCM_INVALID_SHAPE, "dequantize group_size must be a positive integer");
  if (!is_float_dtype(param_dtype) || !is_float_dtype(out_dtype))
    return fail(AFFON_ROCM_INVALID_SHAPE, "dequantize requires f32/bf16 parameters and output");
  const int64_t per_word = 32 / static_cast<int64_t>(bits);
  if (rows <= 0 || columns <= 0 || columns % per_word != 0 || columns % static_cast<int64_t>(group_size) != 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "dequantize columns must divide into complete words and groups");
  uint64_t count = 0;
  if (!mul_ok(static_cast<uint64_t>(rows), static_cast<uint64_t>(columns), &count) || count > (uint64_t(1) << 60))
    return fail(AFFON_ROCM_INVALID_SHAPE, "dequantize size overflows");
  if (packed == nullptr || scales == nullptr || biases == nullptr || out == nullptr)
    return fail(AFFON_ROCM_INVALID_SHAPE, "dequantize buffer is null");
  int status = check_session(session);
  if (status != AFFON_ROCM_OK) return status;
  hipError_t e = affon::dequantize_launch(packed, scales, biases, param_dtype, rows, columns, static_cast<int>(bits),
                                          group_size, out, out_dtype, session->stream);
  if (e != hipSuccess) return hip_fail(e, "dequantize");
  return AFFON_ROCM_OK;
}

static int check_rows(const void* x, int32_t dtype, int64_t rows, int64_t cols, const void* out, const char* op) {
  if (!is_float_dtype(dtype)) return fail(AFFON_ROCM_INVALID_SHAPE, "%s requires an f32 or bf16 tensor", op);
  if (rows <= 0 || cols <= 0) return fail(AFFON_ROCM_INVALID_SHAPE, "%s requires a non-empty rank-two tensor", op);
  uint64_t count = 0;
  // One wave per row (four rows per workgroup) or one thread per element:
  // the grid must stay within 2^31 workgroups.
  if (!mul_ok(static_cast<uint64_t>(rows), static_cast<uint64_t>(cols), &count) || count > (uint64_t(1) << 40) ||
      rows > (int64_t(1) << 32))
    return fail(AFFON_ROCM_INVALID_SHAPE, "%s size overflows", op);
  if (x == nullptr || out == nullptr) return fail(AFFON_ROCM_INVALID_SHAPE, "%s buffer is null", op);
  return AFFON_ROCM_OK;
}

int affon_rocm_rms_norm(affon_rocm_session* session, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                        float epsilon, void* out) {
  clear_error();
  int status = check_rows(x, dtype, rows, cols, out, "rms_norm");
  if (status != AFFON_ROCM_OK) return status;
  // program.ts:578-579: a finite, positive epsilon.
  if (!(epsilon > 0.0f) || epsilon == std::numeric_limits<float>::infinity())
    return fail(AFFON_ROCM_INVALID_SHAPE, "invalid rms_norm options: epsilon must be finite and positive");
  if ((status = check_session(session)) != AFFON_ROCM_OK) return status;
  hipError_t e = affon::rms_norm_launch(x, dtype, rows, cols, epsilon, out, session->stream);
  if (e != hipSuccess) return hip_fail(e, "rms_norm");
  return AFFON_ROCM_OK;
}

int affon_rocm_softmax(affon_rocm_session* session, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                       void* out) {
  clear_error();
  int status = check_rows(x, dtype, rows, cols, out, "softmax");
  if (status != AFFON_ROCM_OK) return status;
  if ((status = check_session(session)) != AFFON_ROCM_OK) return status;
  hipError_t e = affon::softmax_launch(x, dtype, rows, cols, out, session->stream);
  if (e != hipSuccess) return hip_fail(e, "softmax");
  return AFFON_ROCM_OK;
}

int affon_rocm_index_select(affon_rocm_session* session, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                            int32_t axis, const int64_t* index, int64_t count, void* out) {
  clear_error();
  int status = check_rows(x, dtype, rows, cols, out, "index_select");
  if (status != AFFON_ROCM_OK) return status;
  if (axis != 0 && axis != 1) return fail(AFFON_ROCM_INVALID_SHAPE, "index_select axis must be 0 or 1");
  if (count <= 0 || index == nullptr) return fail(AFFON_ROCM_INVALID_SHAPE, "index_select requires indices");
  uint64_t total = 0;
  if (!mul_ok(static_cast<uint64_t>(count), static_cast<uint64_t>(axis == 0 ? cols : rows), &total) ||
      total > (uint64_t(1) << 38))
    return fail(AFFON_ROCM_INVALID_SHAPE, "index_select size overflows");
  if ((status = check_session(session)) != AFFON_ROCM_OK) return status;
  hipError_t e = affon::index_select_launch(x, dtype, rows, cols, axis, index, count, out, session->stream);
  if (e != hipSuccess) return hip_fail(e, "index_select");
  return AFFON_ROCM_OK;
}

// ---- host-pointer drop-in for compute_core_run_quantized_matmul_f32 ----

namespace {

std::mutex g_default_mutex;
affon_rocm_session* g_default_session = nullptr;

struct DeviceBuffer {
  affon_rocm_session* session;
  void* ptr = nullptr;
  explicit DeviceBuffer(affon_rocm_session* s) : session(s) {}
  ~DeviceBuffer() {
    if (ptr != nullptr) {
      hipSetDevice(session->device);
      hipFree(ptr);
    }
  }
};

}  // namespace

int compute_core_run_quantized_matmul_f32(const float* activation, size_t activation_count, const uint32_t* weights,
                                          size_t weight_count, const float* scales, size_t scale_count,
                                          const float* biases, size_t bias_count, float* output, size_t output_count,
                                          size_t rows, size_t depth, size_t columns, size_t bits,
                                          size_t group_size) {
  clear_error();
  // compute_core_cyna.zig:1012-1022, in the same order.
  if (rows == 0 || depth == 0 || columns == 0 || group_size == 0 || (bits != 2 && bits != 4 && bits != 8))
    return fail(AFFON_ROCM_INVALID_SHAPE, "invalid quantized matmul shape");
  const size_t per_word = 32 / bits;
  if (depth % per_word != 0 || depth % group_size != 0)
    return fail(AFFON_ROCM_INVALID_SHAPE, "depth must divide into complete words and groups");
  uint64_t a_count = 0, w_count = 0, g_count = 0, o_count = 0;
  if (!mul_ok(rows, depth, &a_count) || !mul_ok(columns, depth / per_word, &w_count) ||
      !mul_ok(columns, depth / group_size, &g_count) || !mul_ok(rows, columns, &o_count))
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized matmul counts overflow");
  if (activation_count != a_count || weight_count != w_count || scale_count != g_count || bias_count != g_count ||
      output_count != o_count)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized matmul buffer counts do not match the shape");
  if (activation == nullptr || weights == nullptr || scales == nullptr || biases == nullptr || output == nullptr)
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized matmul buffer is null");
  uint64_t a_bytes, w_bytes, g_bytes, o_bytes;
  if (!mul_ok(a_count, 4, &a_bytes) || !mul_ok(w_count, 4, &w_bytes) || !mul_ok(g_count, 4, &g_bytes) ||
      !mul_ok(o_count, 4, &o_bytes))
    return fail(AFFON_ROCM_INVALID_SHAPE, "quantized matmul byte counts overflow");

  std::lock_guard<std::mutex> lock(g_default_mutex);
  if (g_default_session == nullptr) {
    int status = affon_rocm_session_create(0, &g_default_session);
    if (status != AFFON_ROCM_OK) {
      g_default_session = nullptr;
      return AFFON_ROCM_CORE_FAILURE;
    }
  }
  affon_rocm_session* s = g_default_session;
  DeviceBuffer dx(s), dw(s), ds(s), db(s), dout(s);
  int status;
  if ((status = affon_rocm_alloc(s, a_bytes, &dx.ptr)) != AFFON_ROCM_OK ||
      (status = affon_rocm_alloc(s, w_bytes, &dw.ptr)) != AFFON_ROCM_OK ||
      (status = affon_rocm_alloc(s, g_bytes, &ds.ptr)) != AFFON_ROCM_OK ||
      (status = affon_rocm_alloc(s, g_bytes, &db.ptr)) != AFFON_ROCM_OK ||
      (status = affon_rocm_alloc(s, o_bytes, &dout.ptr)) != AFFON_ROCM_OK ||
      (status = affon_rocm_memcpy_h2d(s, dx.ptr, activation, a_bytes)) != AFFON_ROCM_OK ||
      (status = affon_rocm_memcpy_h2d(s, dw.ptr, weights, w_bytes)) != AFFON_ROCM_OK ||
      (status = affon_rocm_memcpy_h2d(s, ds.ptr, scales, g_bytes)) != AFFON_ROCM_OK ||
      (status = affon_rocm_memcpy_h2d(s, db.ptr, biases, g_bytes)) != AFFON_ROCM_OK)
    return AFFON_ROCM_CORE_FAILURE;
  const int64_t K = static_cast<int64_t>(depth), N = static_cast<int64_t>(columns), M = static_cast<int64_t>(rows);
  const int64_t KW = K / static_cast<int64_t>(per_word), G = K / static_cast<int64_t>(group_size);
  affon_rocm_qmm_desc d{};
  d.input = {dx.ptr, a_bytes, 0, {M, K}, {K, 1}, AFFON_ROCM_F32};
  d.packed = {dw.ptr, w_bytes, 0, {N, KW}, {KW, 1}, AFFON_ROCM_U32};
  d.scales = {ds.ptr, g_bytes, 0, {N, G}, {G, 1}, AFFON_ROCM_F32};
  d.biases = {db.ptr, g_bytes, 0, {N, G}, {G, 1}, AFFON_ROCM_F32};
  d.output = static_cast<float*>(dout.ptr);
  d.output_bytes = o_bytes;
  d.bits = static_cast<uint32_t>(bits);
  d.group_size = static_cast<uint32_t>(group_size);
  d.implementation = AFFON_ROCM_IMPL_AUTO;
  d.numerical_policy = AFFON_ROCM_BACKEND_EQUIVALENT;
  if ((status = affon_rocm_quantized_matmul(s, &d)) != AFFON_ROCM_OK) return status == 1 ? 1 : AFFON_ROCM_CORE_FAILURE;
  if ((status = affon_rocm_memcpy_d2h(s, output, dout.ptr, o_bytes)) != AFFON_ROCM_OK) return AFFON_ROCM_CORE_FAILURE;
  return AFFON_ROCM_OK;
}

}  // extern "C"
