// C-ABI entry points of libbased_la.so (declared in include/based_la.h).
//
// Host-side validation happens here, before any launch; argument errors return negative
// LA_ERR_* codes and launch/runtime errors return the positive hipError_t.  Nothing throws
// and nothing is allocated.
#include <math.h>

#include <mutex>

#include "../../include/based_la.h"
#include "la_internal.hpp"

namespace {

bool dtype_ok(int t) { return t == LA_F32 || t == LA_BF16; }
bool finite_f(float x) { return isfinite(x) != 0; }

int check_common(const void* q, const void* k, const void* v, const void* out, int in_dtype, int out_dtype,
                 int B, int H, int N, int d, int dv) {
  if (B < 0 || H < 0 || N < 0 || d < 1 || dv < 1) return LA_ERR_BAD_SHAPE;
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return LA_ERR_BAD_DTYPE;
  if ((long long)B * H * N == 0) return LA_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr) return LA_ERR_NULL_POINTER;
  if ((long long)B * H > 0x7fffffffLL || (long long)N * (d > dv ? d : dv) > 0x7fffffffLL) return LA_ERR_BAD_SHAPE;
  const size_t esz = in_dtype == LA_F32 ? 4 : 2;
  const uintptr_t mask = esz - 1;
  if ((reinterpret_cast<uintptr_t>(q) & mask) || (reinterpret_cast<uintptr_t>(k) & mask) ||
      (reinterpret_cast<uintptr_t>(v) & mask))
    return LA_ERR_BAD_ALIGNMENT;
  const uintptr_t omask = (out_dtype == LA_F32 ? 4 : 2) - 1;
  if (reinterpret_cast<uintptr_t>(out) & omask) return LA_ERR_BAD_ALIGNMENT;
  return LA_OK;
}

}  // namespace

extern "C" {

int la_abi_version(void) { return LA_ABI_VERSION; }

const char* la_status_string(int status) {
  switch (status) {
    case LA_OK: return "success";
    case LA_ERR_NULL_POINTER: return "null tensor pointer";
    case LA_ERR_BAD_SHAPE: return "invalid shape (negative size, d or dv < 1, or a size beyond the 32-bit index range)";
    case LA_ERR_BAD_DTYPE: return "unsupported dtype (expected LA_F32 or LA_BF16)";
    case LA_ERR_BAD_SCALAR: return "invalid scalar argument (scale must be finite and > 0, eps finite and >= 0, window >= 1)";
    case LA_ERR_UNSUPPORTED_DIM: return "unsupported head / value dimension or chunk size for this kernel";
    case LA_ERR_WORKSPACE: return "workspace too small";
    case LA_ERR_NO_DEVICE: return "no HIP device";
    case LA_ERR_BAD_ALIGNMENT: return "tensor pointer not aligned to its element size";
    case LA_ERR_OVERLAP: return "input and output buffers overlap";
    case LA_ERR_SCRATCH_LIMIT: return "shape needs more scratch than the no-allocation entry point's fixed device array";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

size_t la_based_parallel_workspace_bytes(int B, int H, int N, int d, int dv, int in_dtype) {
  if (B < 1 || H < 1 || N < 1 || d < 1 || dv < 1) return 0;
  return la::parallel_workspace_bytes(B * H, N, d, dv, in_dtype == LA_F32);
}

namespace {

bool al(const void* ptr, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(ptr) & (bytes - 1)) == 0; }

// Shared body of the parallel entry points.  stages: 1 = pre-pass only, 2 = main kernel only
// (workspace already holds the pre-pass of this v), 3 = both.
int parallel_entry(const void* q, const void* k, const void* v, int in_dtype, void* out, int out_dtype,
                   float* den_or_null, int B, int H, int N, int d, int dv, float scale, float eps, int normalize,
                   void* workspace, size_t workspace_bytes, void* hip_stream, int stages) {
  int rc = check_common(q, k, v, out, in_dtype, out_dtype, B, H, N, d, dv);
  if (rc != LA_OK) return rc;
  if (d > 128 || dv > 128) return LA_ERR_UNSUPPORTED_DIM;
  if (!finite_f(scale) || !(scale > 0.f) || !finite_f(eps) || eps < 0.f) return LA_ERR_BAD_SCALAR;
  if ((long long)B * H * N == 0) return LA_OK;
  if (den_or_null != nullptr && !al(den_or_null, 4)) return LA_ERR_BAD_ALIGNMENT;
  const size_t need = la::parallel_workspace_bytes(B * H, N, d, dv, in_dtype == LA_F32);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return LA_ERR_WORKSPACE;
  if (need > 0 && !al(workspace, 16)) return LA_ERR_BAD_ALIGNMENT;
  // the packed kernels copy q, k, v^T rows 16 bytes at a time and store out 8 bytes at a time;
  // misaligned tensors of a packed shape run the register-staged kernel, which needs the
  // pre-pass and the main kernel in one call
  const bool aligned = al(q, 16) && al(k, 16) && al(v, 8) && al(out, 16);
  if (la::parallel_packed_shape(d, dv, in_dtype == LA_F32) && stages != 3 && !aligned) return LA_ERR_BAD_ALIGNMENT;
  la::ParallelArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.den = den_or_null;
  a.workspace = need > 0 ? workspace : nullptr;
  a.workspace_bytes = need > 0 ? workspace_bytes : 0;
  a.packed_aligned = aligned;
  // fp32 inputs have no pre-pass: a pack-only call does nothing, a main-only call is the whole call
  a.stages = need > 0 ? stages : (stages & 2 ? 3 : 0);
  a.BH = B * H;
  a.N = N;
  a.d = d;
  a.dv = dv;
  a.scale = scale;
  a.eps = eps;
  a.normalize = normalize != 0;
  a.in_f32 = in_dtype == LA_F32;
  a.out_f32 = out_dtype == LA_F32;
  if (a.stages == 0) return LA_OK;
  return la::launch_based_parallel(a, static_cast<hipStream_t>(hip_stream));
}

}  // namespace

int la_based_parallel_fwd(const void* q, const void* k, const void* v, int in_dtype, void* out, int out_dtype,
                          float* den_or_null, int B, int H, int N, int d, int dv, float scale, float eps,
                          int normalize, void* workspace, size_t workspace_bytes, void* hip_stream) {
  return parallel_entry(q, k, v, in_dtype, out, out_dtype, den_or_null, B, H, N, d, dv, scale, eps, normalize,
                        workspace, workspace_bytes, hip_stream, 3);
}

int la_based_parallel_pack(const void* k, const void* v, int in_dtype, int B, int H, int N, int d, int dv,
                           void* workspace, size_t workspace_bytes, void* hip_stream) {
  // q and out are not touched by the pre-pass; k stands in for them in the shared checks
  return parallel_entry(k, k, v, in_dtype, const_cast<void*>(k), in_dtype, nullptr, B, H, N, d, dv, 1.0f, 0.f, 1,
                        workspace, workspace_bytes, hip_stream, 1);
}

int la_based_parallel_fwd_packed(const void* q, const void* k, const void* v, int in_dtype, void* out,
                                 int out_dtype, float* den_or_null, int B, int H, int N, int d, int dv, float scale,
                                 float eps, int normalize, void* workspace, size_t workspace_bytes,
                                 void* hip_stream) {
  return parallel_entry(q, k, v, in_dtype, out, out_dtype, den_or_null, B, H, N, d, dv, scale, eps, normalize,
                        workspace, workspace_bytes, hip_stream, 2);
}

size_t la_based_chunked_workspace_bytes(int B, int H, int N, int d, int dv, int chunk) {
  if (B < 1 || H < 1 || N < 1 || d < 1 || dv < 1 || chunk < 1) return 0;
  const size_t b16 = la::chunked_workspace_bytes(B * H, N, d, dv, chunk);
  const size_t f32 = la::general_chunked_bytes(B * H, N, d, dv, true);
  if (b16 == (size_t)-1 || f32 == (size_t)-1) return b16 == (size_t)-1 ? f32 : b16;
  return b16 > f32 ? b16 : f32;   // enough for either input type
}

size_t la_based_chunked_workspace_bytes_dt(int B, int H, int N, int d, int dv, int chunk, int in_dtype) {
  if (B < 1 || H < 1 || N < 1 || d < 1 || dv < 1 || chunk < 1) return 0;
  if (in_dtype == LA_F32) return la::general_chunked_bytes(B * H, N, d, dv, true);
  if (in_dtype != LA_BF16) return (size_t)-1;
  return la::chunked_workspace_bytes(B * H, N, d, dv, chunk);
}

int la_based_chunked_chunk_used(int chunk) {
  if (chunk < 1) return LA_ERR_BAD_SHAPE;
  return la::chunked_chunk_tokens();
}

static int chunked_common(const void* q, const void* k, const void* v, int in_dtype, void* out, int out_dtype, int B,
                          int H, int N, int d, int dv, int chunk, float scale, float eps, int normalize,
                          void* workspace, size_t workspace_bytes, const float* state_in, long long prev_tokens,
                          float* state_out_or_null, void* hip_stream, float* den_out = nullptr) {
  int rc = check_common(q, k, v, out, in_dtype, out_dtype, B, H, N, d, dv);
  if (rc != LA_OK) return rc;
  if (!finite_f(scale) || !(scale > 0.f) || !finite_f(eps) || eps < 0.f) return LA_ERR_BAD_SCALAR;
  if (chunk < 1) return LA_ERR_BAD_SHAPE;
  if ((long long)B * H * N == 0) return LA_OK;
  const size_t need = la::chunked_scratch_bytes(B * H, N, d, dv, state_in != nullptr, in_dtype == LA_F32);
  if (need == (size_t)-1) return LA_ERR_UNSUPPORTED_DIM;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return LA_ERR_WORKSPACE;
  if (need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 15)) return LA_ERR_BAD_ALIGNMENT;   // 16-byte accesses
  if (state_out_or_null != nullptr && (reinterpret_cast<uintptr_t>(state_out_or_null) & 3)) return LA_ERR_BAD_ALIGNMENT;
  if (state_in != nullptr) {
    if (reinterpret_cast<uintptr_t>(state_in) & 3) return LA_ERR_BAD_ALIGNMENT;
    if (prev_tokens < 0) return LA_ERR_BAD_SCALAR;
    // the last segment writes state_out while other segments may still read state_in
    const char* i0 = reinterpret_cast<const char*>(state_in);
    const char* o0 = reinterpret_cast<const char*>(state_out_or_null);
    const size_t bytes = (size_t)B * H * 153 * (size_t)(dv + 1) * 4;
    if (o0 != nullptr && i0 < o0 + bytes && o0 < i0 + bytes) return LA_ERR_OVERLAP;
  }
  if (den_out != nullptr && (reinterpret_cast<uintptr_t>(den_out) & 3)) return LA_ERR_BAD_ALIGNMENT;
  la::ChunkedArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.den_out = den_out;
  a.state_out = state_out_or_null;
  a.state_in = state_in;
  a.prev_tokens = state_in != nullptr ? prev_tokens : 0;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.BH = B * H;
  a.N = N;
  a.d = d;
  a.dv = dv;
  a.chunk = chunk;
  a.scale = scale;
  a.eps = eps;
  a.normalize = normalize != 0;
  a.in_f32 = in_dtype == LA_F32;
  a.out_f32 = out_dtype == LA_F32;
  return la::launch_based_chunked(a, static_cast<hipStream_t>(hip_stream));
}

int la_based_layer_fwd(const void* q, const void* k, const void* v, const void* q_sw, const void* k_sw,
                       int in_dtype, void* out, int out_dtype, int B, int H, int N, int d, int dv, int d_sw,
                       int window, float scale, float scale_sw, float eps, void* workspace,
                       size_t workspace_bytes, void* hip_stream) {
  int rc = check_common(q, k, v, out, in_dtype, out_dtype, B, H, N, d, dv);
  if (rc != LA_OK) return rc;
  if (q_sw == nullptr || k_sw == nullptr) return LA_ERR_NULL_POINTER;
  if (in_dtype != LA_BF16) return LA_ERR_BAD_DTYPE;
  if (!la::layer_fused_shape(d, dv, d_sw, window)) return LA_ERR_UNSUPPORTED_DIM;
  if (!finite_f(scale) || !(scale > 0.f) || !finite_f(scale_sw) || !(scale_sw > 0.f) || !finite_f(eps) || eps < 0.f)
    return LA_ERR_BAD_SCALAR;
  if ((long long)B * H * N == 0) return LA_OK;
  if (!al(q, 16) || !al(k, 16) || !al(v, 16) || !al(q_sw, 16) || !al(k_sw, 16) || !al(out, 16))
    return LA_ERR_BAD_ALIGNMENT;
  const size_t need = la::chunked_scratch_bytes(B * H, N, d, dv, false, false);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return LA_ERR_WORKSPACE;
  if (need > 0 && !al(workspace, 16)) return LA_ERR_BAD_ALIGNMENT;
  la::LayerArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.qsw = q_sw;
  a.ksw = k_sw;
  a.out = out;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.BH = B * H;
  a.N = N;
  a.d = d;
  a.dv = dv;
  a.dsw = d_sw;
  a.window = window;
  a.scale = scale;
  a.scale_sw = scale_sw;
  a.eps = eps;
  a.out_f32 = out_dtype == LA_F32;
  return la::launch_based_layer(a, static_cast<hipStream_t>(hip_stream));
}

int la_based_chunked_fwd(const void* q, const void* k, const void* v, int in_dtype, void* out, int out_dtype, int B,
                         int H, int N, int d, int dv, int chunk, float scale, float eps, int normalize,
                         void* workspace, size_t workspace_bytes, float* state_out_or_null, void* hip_stream) {
  return chunked_common(q, k, v, in_dtype, out, out_dtype, B, H, N, d, dv, chunk, scale, eps, normalize, workspace,
                        workspace_bytes, nullptr, 0, state_out_or_null, hip_stream);
}

int la_based_chunked_fwd_num_den(const void* q, const void* k, const void* v, int in_dtype, float* num_out,
                                 float* den_out, int B, int H, int N, int d, int dv, int chunk, float scale,
                                 void* workspace, size_t workspace_bytes, void* hip_stream) {
  if (den_out == nullptr && (long long)B * H * N != 0) return LA_ERR_NULL_POINTER;
  return chunked_common(q, k, v, in_dtype, num_out, LA_F32, B, H, N, d, dv, chunk, scale, 0.0f, 0, workspace,
                        workspace_bytes, nullptr, 0, nullptr, hip_stream, den_out);
}

}  // extern "C"

// ---- no-allocation variant of la_based_chunked_fwd
//
// The chunked kernels' scratch (per (head, segment) state increments and their prefixes) lives
// in a file-scope device array instead of a caller workspace.  Host code never passes the
// array's name to a kernel: its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and kept in g_scratch_ptr.  Every call on a
// device shares that device's array; the kernels write every scratch word they read before
// reading it, so nothing needs clearing between calls, but calls that overlap on one device
// (different streams, or host threads) race on it.
namespace {

static __device__ __align__(256) unsigned char scratch[LA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the device that owns `stream` (the current device for the null
// stream), looked up on the first call for that device.
int scratch_for_stream(hipStream_t stream, void** out) {
  int dev = -1;
  if (stream != nullptr) {
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return LA_ERR_NO_DEVICE;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return LA_ERR_NO_DEVICE;
  }
  if (dev < 0 || dev >= kMaxDevices) return LA_ERR_NO_DEVICE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return LA_ERR_NO_DEVICE;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return LA_ERR_NO_DEVICE;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return LA_ERR_NO_DEVICE;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LA_OK;
}

}  // namespace

extern "C" {

int la_based_chunked_fwd_noalloc(const void* q, const void* k, const void* v, int in_dtype, void* out,
                                 int out_dtype, int B, int H, int N, int d, int dv, int chunk, float scale,
                                 float eps, int normalize, float* state_out_or_null, void* hip_stream) {
  int rc = check_common(q, k, v, out, in_dtype, out_dtype, B, H, N, d, dv);
  if (rc != LA_OK) return rc;
  if (chunk < 1) return LA_ERR_BAD_SHAPE;
  if ((long long)B * H * N == 0) return LA_OK;
  const size_t need = la::chunked_scratch_bytes(B * H, N, d, dv, false, in_dtype == LA_F32);
  if (need == (size_t)-1) return LA_ERR_UNSUPPORTED_DIM;
  if (need > (size_t)LA_NOALLOC_SCRATCH_BYTES) return LA_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_for_stream(static_cast<hipStream_t>(hip_stream), &ws);
    if (rc != LA_OK) return rc;
  }
  return chunked_common(q, k, v, in_dtype, out, out_dtype, B, H, N, d, dv, chunk, scale, eps, normalize, ws,
                        need > 0 ? (size_t)LA_NOALLOC_SCRATCH_BYTES : 0, nullptr, 0, state_out_or_null, hip_stream);
}

int la_based_chunked_fwd_continue(const void* q, const void* k, const void* v, int in_dtype, void* out,
                                  int out_dtype, int B, int H, int N, int d, int dv, int chunk, float scale,
                                  float eps, int normalize, void* workspace, size_t workspace_bytes,
                                  const float* state_in, long long prev_tokens, float* state_out_or_null,
                                  void* hip_stream) {
  if (state_in == nullptr && (long long)B * H * N != 0) return LA_ERR_NULL_POINTER;
  return chunked_common(q, k, v, in_dtype, out, out_dtype, B, H, N, d, dv, chunk, scale, eps, normalize, workspace,
                        workspace_bytes, state_in, prev_tokens, state_out_or_null, hip_stream);
}

size_t la_identity_workspace_bytes(int B, int H, int N, int d, int dv) {
  if (B < 0 || H < 0 || N < 0) return 0;
  return la::identity_workspace_bytes(B * H, N, d, dv);
}

int la_identity_linear_fwd(const void* q, const void* k, const void* v, int in_dtype, void* out, int out_dtype, int B,
                           int H, int N, int d, int dv, float scale, void* workspace, size_t workspace_bytes,
                           void* hip_stream) {
  int rc = check_common(q, k, v, out, in_dtype, out_dtype, B, H, N, d, dv);
  if (rc != LA_OK) return rc;
  if (in_dtype != LA_BF16) return LA_ERR_BAD_DTYPE;
  if (!la::identity_shape(d, dv)) return LA_ERR_UNSUPPORTED_DIM;
  if (!finite_f(scale)) return LA_ERR_BAD_SCALAR;
  if ((long long)B * H * N == 0) return LA_OK;
  if ((size_t)N * (size_t)(d > dv ? d : dv) * 2 >= ((size_t)1 << 31)) return LA_ERR_BAD_SHAPE;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
        reinterpret_cast<uintptr_t>(out)) & 15) != 0)
    return LA_ERR_BAD_ALIGNMENT;
  const size_t need = la::identity_workspace_bytes(B * H, N, d, dv);
  if (workspace == nullptr || workspace_bytes < need) return LA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) & 15) return LA_ERR_BAD_ALIGNMENT;
  la::IdentityArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.workspace = workspace;
  a.BH = B * H;
  a.N = N;
  a.d = d;
  a.dv = dv;
  a.scale = scale;
  a.out_f32 = out_dtype == LA_F32;
  return la::launch_identity(a, static_cast<hipStream_t>(hip_stream));
}

static int decode_common(const void* q, const void* k, const void* v, int in_dtype, float* state, void* out,
                         int out_dtype, int B, int H, int d, int dv, float eps, int normalize, bool with_ws,
                         void* workspace, size_t workspace_bytes, void* hip_stream) {
  int rc = check_common(q, k, v, out, in_dtype, out_dtype, B, H, 1, d, dv);
  if (rc != LA_OK) return rc;
  if (!la::decode_shape(d, dv)) return LA_ERR_UNSUPPORTED_DIM;
  if (!finite_f(eps) || eps < 0.f) return LA_ERR_BAD_SCALAR;
  if ((long long)B * H == 0) return LA_OK;
  if (state == nullptr) return LA_ERR_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(state) & 3) return LA_ERR_BAD_ALIGNMENT;
  la::DecodeArgs a{};
  if (with_ws) {
    const size_t need = la::decode_workspace_bytes((long long)B * H, d, dv);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return LA_ERR_WORKSPACE;
    if (need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 3)) return LA_ERR_BAD_ALIGNMENT;
    a.workspace = need > 0 ? workspace : nullptr;
  }
  a.q = q;
  a.k = k;
  a.v = v;
  a.state = state;
  a.out = out;
  a.BH = B * H;
  a.d = d;
  a.dv = dv;
  a.eps = eps;
  a.normalize = normalize != 0;
  a.in_f32 = in_dtype == LA_F32;
  a.out_f32 = out_dtype == LA_F32;
  return la::launch_decode_step(a, static_cast<hipStream_t>(hip_stream));
}

int la_based_decode_step(const void* q, const void* k, const void* v, int in_dtype, float* state, void* out,
                         int out_dtype, int B, int H, int d, int dv, float eps, int normalize, void* hip_stream) {
  return decode_common(q, k, v, in_dtype, state, out, out_dtype, B, H, d, dv, eps, normalize, false, nullptr, 0,
                       hip_stream);
}

size_t la_based_decode_workspace_bytes(int B, int H, int d, int dv) {
  if (B < 0 || H < 0 || !la::decode_shape(d, dv)) return 0;
  return la::decode_workspace_bytes((long long)B * H, d, dv);
}

int la_based_decode_step_ws(const void* q, const void* k, const void* v, int in_dtype, float* state, void* out,
                            int out_dtype, int B, int H, int d, int dv, float eps, int normalize, void* workspace,
                            size_t workspace_bytes, void* hip_stream) {
  return decode_common(q, k, v, in_dtype, state, out, out_dtype, B, H, d, dv, eps, normalize, true, workspace,
                       workspace_bytes, hip_stream);
}

static int sliding_common(const void* q, const void* k, const void* v, int in_dtype, bool with_addend,
                          const float* addend, void* out, int out_dtype, int B, int H, int N, int d, int dv,
                          int window, float scale, void* hip_stream) {
  int rc = check_common(q, k, v, out, in_dtype, out_dtype, B, H, N, d, dv);
  if (rc != LA_OK) return rc;
  if (d > 128 || dv > 128) return LA_ERR_UNSUPPORTED_DIM;
  if (window < 1 || !finite_f(scale) || !(scale > 0.f)) return LA_ERR_BAD_SCALAR;
  if ((long long)B * H * N == 0) return LA_OK;
  if (with_addend && addend == nullptr) return LA_ERR_NULL_POINTER;
  if (with_addend && (reinterpret_cast<uintptr_t>(addend) & 15)) return LA_ERR_BAD_ALIGNMENT;
  la::SlidingArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.addend = addend;
  a.BH = B * H;
  a.N = N;
  a.d = d;
  a.dv = dv;
  a.window = window;
  a.scale = scale;
  a.in_f32 = in_dtype == LA_F32;
  a.out_f32 = out_dtype == LA_F32;
  return la::launch_sliding_window(a, static_cast<hipStream_t>(hip_stream));
}

int la_sliding_window_fwd(const void* q, const void* k, const void* v, int in_dtype, void* out, int out_dtype, int B,
                          int H, int N, int d, int dv, int window, float scale, void* hip_stream) {
  return sliding_common(q, k, v, in_dtype, false, nullptr, out, out_dtype, B, H, N, d, dv, window, scale,
                        hip_stream);
}

int la_sliding_window_fwd_add(const void* q, const void* k, const void* v, int in_dtype, const float* addend,
                              void* out, int out_dtype, int B, int H, int N, int d, int dv, int window, float scale,
                              void* hip_stream) {
  return sliding_common(q, k, v, in_dtype, true, addend, out, out_dtype, B, H, N, d, dv, window, scale, hip_stream);
}

int la_taylor_feature_map(const void* x, int in_dtype, void* out, int out_dtype, long long rows, int d,
                          void* hip_stream) {
  if (rows < 0 || d < 1) return LA_ERR_BAD_SHAPE;
  if (d > 128) return LA_ERR_UNSUPPORTED_DIM;
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return LA_ERR_BAD_DTYPE;
  if (rows == 0) return LA_OK;
  if (x == nullptr || out == nullptr) return LA_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(x) & (in_dtype == LA_F32 ? 3 : 1)) ||
      (reinterpret_cast<uintptr_t>(out) & (out_dtype == LA_F32 ? 3 : 1)))
    return LA_ERR_BAD_ALIGNMENT;
  const long long F = 1 + (long long)d + (long long)d * (d + 1) / 2;
  if (rows > (1LL << 40) / F) return LA_ERR_BAD_SHAPE;   // rows * F elements, without overflow
  la::FeatureMapArgs a{};
  a.x = x;
  a.out = out;
  a.rows = rows;
  a.d = d;
  a.in_f32 = in_dtype == LA_F32;
  a.out_f32 = out_dtype == LA_F32;
  return la::launch_feature_map(a, static_cast<hipStream_t>(hip_stream));
}

}  // extern "C"
