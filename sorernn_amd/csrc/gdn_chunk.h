// Internal interface between the two kernels of the chunked prefill and its C-ABI entry point.
//
// The prefill runs as two launches on the caller's stream:
//   1. gated_delta_chunk_prep_kernel (gdn_chunk_prep.hip): for every 64-token chunk and value head,
//      the inverse T = (I + A)^-1 of the chunk's unit lower-triangular system, written to the
//      workspace as fp16 rows of T - I. Chunks are independent, so this kernel is fully parallel.
//   2. gated_delta_chunk_kernel (gdn_chunk.hip): the sequential state recurrence over the chunks
//      of each sequence, reading T from the workspace.
// With cu_seqlens, a one-block gated_delta_chunk_index_kernel first writes the number of chunks
// before every sequence (the prep kernel's chunk -> sequence map) into the workspace.
//
// Workspace (caller-owned, gdn_chunk_workspace_size bytes):
//   [0, tbytes)                T - I rows: fp16 [B*T][HV][64], row t of the chunk holding token t,
//                              columns in tok_col order (gdn_mfma.h)
//   then, with cu_seqlens only: int32 chunk_first[N + 1] and int32 order[N] (256-byte aligned each)
#pragma once

#include "gdn_mfma.h"

namespace gdn {

struct ChunkPrepParams {
  const void *k, *g, *beta;
  f16* tw;                 // T - I rows (workspace)
  const void* cu;
  const int* chunk_first;  // with cu only
  const int* order;        // with cu only: sequences by length, longest first (written by the index kernel)
  int cu_i32;
  int64_t T, H, HV, N;
  int dg, db;
  unsigned flags;
  const float *A_log, *dt_bias;
  int64_t items;           // set by launch_chunk_prep: chunks per value head (an upper bound with cu)
};

inline int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }
inline int64_t chunk_t_bytes(int64_t tokens, int64_t HV) { return align256(tokens * HV * kC * 2); }

// Launches the index kernel (with cu) and the prep kernel; returns a GDN status.
int launch_chunk_prep(const ChunkPrepParams& p, int64_t B, int64_t K, hipStream_t s);
// The index kernel sorts sequences longest first for up to kOrderMax of them (identity order above).
constexpr int kOrderMax = 2048;
// Compute units of the device that runs stream s (cached per device).
int device_compute_units(hipStream_t s);
// Launches the index kernel only (with cu): chunk_first and the longest-first order.
int launch_chunk_index(const void* cu, int cu_i32, int64_t N, int* chunk_first, int* order, hipStream_t s);

// The cooperative prefill (gdn_chunk_coop.hip): one launch for K = V = 128 inference calls. The
// four 32-column slices of a (sequence, head) chain share the per-chunk P, T/A blocks and gate
// terms through a ring in the workspace; the sync words must be zero at launch (the launcher
// clears them with a fill kernel first).
struct CoopArgs {
  const void *q, *k, *v, *g, *beta;
  const float* h0;
  void* o;
  float* ht;
  const void* cu;
  const int* order;
  int cu_i32;
  int64_t T, H, HV, N;
  int dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
  char* ring;
  unsigned* sync;
  unsigned* range_flag;
  unsigned* err;
};
int coop_ring_slots(int64_t T);                    // ring slots per chain for sequences of <= T tokens
int64_t coop_ring_bytes(int64_t chains, int64_t T);
int64_t coop_sync_bytes(int64_t chains);  // includes one error word after the chains' sync words
int launch_chunk_coop(const CoopArgs& a, hipStream_t s);
// Zeroes `words` 32-bit words with a fill kernel (captured graphs clear them on every replay).
int launch_fill_zero(unsigned* w, int64_t words, hipStream_t s);
// Gated RMSNorm of bf16 rows (gdn_norm.hip): y = x rstd w silu(gate), or with split the norm and
// silu(gate) rounded separately (o_norm(o) * F.silu(gate)); y may be x. Returns a GDN status.
int gdn_internal_rms_norm_gated(const void* x, const void* gate, const float* w, void* y, int64_t rows, int64_t D,
                                float eps, int split, hipStream_t s);

}  // namespace gdn
