// Host-side launch descriptors shared between the C-ABI layer (capi.hip) and the kernel
// translation units.  Internal to libbased_la.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace la {

struct ParallelArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* den;          // optional, (BH, N) fp32, den without eps
  void* workspace;     // parallel_workspace_bytes() of scratch (bf16 inputs)
  size_t workspace_bytes;
  bool packed_aligned; // q, k, out 16-byte and v 8-byte aligned: the packed kernels may run
  int stages;          // packed path: 1 = pre-pass (pack V), 2 = main kernel, 3 = both
  int BH, N, d, dv;
  float scale, eps;
  bool normalize;
  bool in_f32, out_f32;
};

struct SlidingArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const float* addend;   // optional fp32 (BH, N, dv) added to the output (may alias an fp32 out)
  int BH, N, d, dv, window;
  float scale;
  bool in_f32, out_f32;
};

struct ChunkedArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* state_out;    // optional, (BH, F, dv + 1) fp32
  const float* state_in;   // optional initial state, same layout
  long long prev_tokens;   // tokens summarised by state_in
  float* den_out;      // optional, (BH, N) fp32: each row's denominator without eps
  void* workspace;
  size_t workspace_bytes;
  int BH, N, d, dv, chunk;
  float scale, eps;
  bool normalize;
  bool in_f32, out_f32;
};

struct LayerArgs {
  const void* q;       // linear branch (d = 16)
  const void* k;
  const void* v;
  const void* qsw;     // softmax branch (dsw)
  const void* ksw;
  void* out;
  void* workspace;     // chunked_workspace_bytes()
  size_t workspace_bytes;
  int BH, N, d, dv, dsw, window;
  float scale, scale_sw, eps;
  bool out_f32;
};

struct IdentityArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  void* workspace;     // identity_workspace_bytes() bytes, 16-byte aligned
  int BH, N, d, dv;
  float scale;
  bool out_f32;
};

struct DecodeArgs {
  const void* q;       // (BH, d)
  const void* k;       // (BH, d)
  const void* v;       // (BH, dv)
  float* state;        // (BH, F, dv + 1) fp32, updated in place
  void* out;           // (BH, dv)
  void* workspace;     // decode_workspace_bytes(BH, d, dv) bytes, or null: one work-group per head
  int BH, d, dv;
  float eps;
  bool normalize, in_f32, out_f32;
};

struct FeatureMapArgs {
  const void* x;
  void* out;
  long long rows;
  int d;
  bool in_f32, out_f32;
};

// Each launcher validates what only it knows (supported tile shapes), launches on `stream`
// and returns 0, a negative LA_ERR_* code, or a positive hipError_t.
int launch_based_parallel(const ParallelArgs& a, hipStream_t stream);
size_t parallel_workspace_bytes(int BH, int N, int d, int dv, bool in_f32);
int f32_split_slots(int BH, int N);                         // fp32 key split: slots per head, or 0
int f32_x6_split_parts(int BH, int N, int d, int dv);       // fp32 three-term key split: parts, or 0
size_t f32_split_workspace_bytes(int BH, int N, int d, int dv);   // partials of either split (or 0)
bool parallel_packed_shape(int d, int dv, bool in_f32);   // shapes of the packed (pre-pass) kernel
int launch_sliding_window(const SlidingArgs& a, hipStream_t stream);
size_t chunked_workspace_bytes(int BH, int N, int d, int dv, int chunk);
int chunked_chunk_tokens();   // tokens per chunk of the chunked kernels
// Bytes of scratch the chunked kernels actually use for this call: 0 when the sequence is one
// segment and there is no initial state, (size_t)-1 for unsupported shapes.
size_t chunked_scratch_bytes(int BH, int N, int d, int dv, bool with_state, bool in_f32);
int launch_based_chunked(const ChunkedArgs& a, hipStream_t stream);
// Segment-state chunked path for the shapes the recurrence kernel does not take (d <= 64,
// dv <= 128; bf16 in chunked_general.hip, fp32 in chunked_general_f32.hip).
bool general_chunked_shape(int d, int dv, bool in_f32);
size_t general_chunked_bytes(int BH, int N, int d, int dv, bool in_f32);   // workspace, (size_t)-1 if unsupported
int launch_general_chunked(const ChunkedArgs& a, hipStream_t stream);
size_t general_chunked_f32_bytes(int BH, int N, int d, int dv);
int launch_general_chunked_f32(const ChunkedArgs& a, hipStream_t stream);
bool layer_fused_shape(int d, int dv, int dsw, int window);   // shapes of chunked_layer_kernel
int launch_based_layer(const LayerArgs& a, hipStream_t stream);
int launch_feature_map(const FeatureMapArgs& a, hipStream_t stream);
int device_cu_count();   // compute units of the current device (256 when the query fails)
bool identity_shape(int d, int dv);
size_t identity_workspace_bytes(int BH, int N, int d, int dv);
int launch_identity(const IdentityArgs& a, hipStream_t stream);
bool decode_shape(int d, int dv);
int launch_decode_step(const DecodeArgs& a, hipStream_t stream);
size_t decode_workspace_bytes(long long BH, int d, int dv);

// Work-group order for causal query blocks: heaviest (last) blocks first over all the heads an
// XCD owns, so that greedy dispatch as slots free up balances the causal triangle (a head-major
// order leaves the last heads' long blocks for the end).  When the head count is a multiple of
// the 8 XCDs each XCD owns whole heads, so a head's K/V prefix is only read through one L2.
// Work-groups are dispatched to XCDs round-robin by work-group id.
//
// pair_cus > 0 (the CUs of one XCD, for kernels that hold two work-groups per CU): within an
// XCD the first pair_cus work-groups go one per CU and the next pair_cus to the same CUs in the
// same order (per-work-group hardware ids on MI355X), and of two work-groups sharing a CU the
// older issues about twice as fast.  The second half of that first round then takes its jobs in
// reverse order, so that the CU holding the heaviest block also holds the lightest of the round
// and every CU starts with the same work: B2 H16 N8192 d16 dv64 whole forward 189.2 -> 185.4 us,
// B2 H16 N4096 68.7 -> 66.6 us, B1 H16 N8192 115.5 -> 112.7 us (one process).
__host__ __device__ __forceinline__ void map_causal_block(int wg, int BH, int nqb, int& bh, int& qb, int pair_cus = 0) {
  if ((BH & 7) == 0) {
    const int x = wg & 7, hpx = BH >> 3;
    int slot = wg >> 3;
    if (pair_cus > 0 && hpx * nqb >= 2 * pair_cus && slot >= pair_cus && slot < 2 * pair_cus)
      slot = 3 * pair_cus - 1 - slot;
    const int r = slot / hpx;
    qb = nqb - 1 - r;
    bh = (slot - r * hpx) * 8 + x;
  } else {
    const int r = wg / BH;
    qb = nqb - 1 - r;
    bh = wg - r * BH;
  }
}

}  // namespace la
