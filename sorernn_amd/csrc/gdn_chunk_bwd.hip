// Backward of the chunked gated delta rule for gfx950 (training through chunk_gated_delta_rule).
//
// Per chunk of c <= 64 tokens the forward computes (gam = in-chunk cumsum of g, a = e^gam,
// r = e^{gam_c - gam}, E_tj = e^{gam_t - gam_j}, T = (I + A)^-1 with A_tj = beta_t E_tj k_t.k_j, j < t):
//   Y = K S,  X = diag(beta) V - diag(beta a) Y,  Delta = T X,
//   O = scale (diag(a) Q S + P Delta),  P = (Q K^T) o E (j <= t),  S' = e^{gam_c} S + K^T diag(r) Delta.
// Given dO and dS' (the gradient of the state leaving the chunk), its backward is
//   dDelta = scale P^T dO + diag(r) K dS',   dX = T^T dDelta,   dV = diag(beta) dX,
//   dS     = e^{gam_c} dS' + scale Q^T diag(a) dO - K^T diag(beta a) dX            (to the previous chunk)
//   dA     = -strict(dX Delta^T),  dG = diag(beta) dA o E,  dQK = scale (dO Delta^T) o E (j <= t)
//   dQ     = scale diag(a) dO S^T + dQK K
//   dK     = diag(r) Delta dS'^T - diag(beta a) dX S^T + dQK^T Q + (dG + dG^T) K
//   dbeta  = rowsum(dA o E o KK^T) + rowsum((V - diag(a) Y) o dX)
//   dgam   = rowsum(Q o dQ_S) - rowsum(diag(beta a) dX o Y) - diag(r) rowsum(K dS' o Delta)
//            + rowsum(Pi) - colsum(Pi),  Pi = dG o KK^T + dQK o QK^T
//            (+ e^{gam_c} <S, dS'> + sum_t r_t (K dS')_t . Delta_t at the chunk's last position),
//   dg     = reverse in-chunk cumsum of dgam.
// oracle/gdn_oracle.py::_chunk_segment_bwd restates the same algebra in fp64 (pinned there against
// autograd through the token recurrence of sore/model/gdn_ref.py:11-22).
//
// Four launches on the caller's stream, after a forward that saved the state entering every chunk
// (gdn_chunk_fwd_train):
//   1. gated_delta_chunk_bwd_prep_kernel, per (chunk, value head): (T - I)^T rows (bf16, for
//      launches 2 and 3, which read the forward's fp16 T - I rows where they need T - I itself)
//      and G1 = T^T (scale P^T dO), the state-independent part of dX
//      (bf16, chunk-blocked [chunk][value head][value column][64 tokens], so that a lane's four
//      adjacent tokens of one column are one 8-byte access in every kernel that touches it).
//   2. gated_delta_chunk_bwd_state_kernel, per (sequence, value head, 32 value columns): the reverse
//      recurrence dS <- e^{gam_c} dS + K^T (-beta a dX) + Q^T (scale a dO) with
//      dX = G1 + T^T (r o K dS), over the chunks from last to first; it stores dS' of every chunk
//      and the initial state's gradient.
//   3. gated_delta_chunk_bwd_grad_kernel, per (chunk, q/k head): everything else, from the saved
//      S, the stored dS' and the chunk's tiles; the value heads that share a q/k head are summed
//      in registers (GVA), and the L2-norm, gate and sigmoid backwards are applied on the way out.
//   4. gated_delta_gate_param_grad_kernel (in-kernel gate only): dA_log and ddt_bias per head from
//      the per-chunk partial sums.
// MFMA operands are bf16 (v_mfma_f32_16x16x32_bf16) with fp32 accumulation: gradients span a range
// of magnitudes that fp16 cannot hold (a mean loss over 10^8 outputs gives dO ~ 1e-8).

#include "gdn_chunk.h"

namespace gdn {

struct ChunkBwdParams {
  const void *q, *k, *v, *g, *beta, *dout;
  const float* dht;   // gradient of the final state [N][HV][K][V], or null
  const bf16* hs;     // state entering each chunk, bf16 [chunks][HV][V][K] (forward output, transposed)
  const f16* tw;      // the forward's T - I rows (fp16, tok_col columns)
  bf16* tnt;          // (T - I)^T rows, bf16 [tokens][HV][64]                   (workspace)
  bf16* g1;           // G1 = T^T (scale P^T dO), bf16 [chunks][HV][V][64 tokens] (workspace)
  bf16* dhs;          // gradient of the state leaving each chunk, bf16 [chunks][HV][V][K]   (workspace)
  float* gate_part;   // per-chunk partial sums of dA_log and ddt_bias [chunks][HV][2] (workspace)
  const void* cu;
  const int* chunk_first;
  int cu_i32;
  int64_t T, H, HV, N;
  int dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
  void *dq, *dk, *dv, *dgate, *dbeta;
  float *dh0, *dA_log, *ddt_bias;
};

constexpr int kCPb = 72;  // bf16 pitch of [*][64] tiles (144 B rows: row and transposed reads conflict-free)
template <int D>
constexpr int row_pitch() { return D == 128 ? D + 16 : D + 8; }  // bf16 pitch of [*][D] tiles

// ---------------------------------------------------------------- fragments from row-major bf16 LDS tiles
// frag_row: lane (g, i) reads M[r0 + i][c0 + 8g .. c0 + 8g + 7] -- the A operand for rows r0.. of M
// with the contraction along M's rows, or the B operand of M^T.
__device__ __forceinline__ bf16x8 frag_row(const bf16* M, int pitch, int r0, int c0, int lane) {
  return ld8(M + (r0 + (lane & 15)) * pitch + c0 + 8 * (lane >> 4));
}
// frag_col: lane (g, i) gets M[r0 + 8g + j][c0 + i], j = 0..7 (two ds_read_b64_tr_b16: lane 4m + q
// reads row r0 + 8g + m (then + 4) at columns c0 + 4q..+3) -- the B operand of M (contraction
// along M's rows, output columns c0..) or the A operand of M^T.
__device__ __forceinline__ bf16x8 frag_col(const bf16* M, int pitch, int r0, int c0, int lane) {
  const int g = lane >> 4, li = lane & 15;
  const bf16* p0 = M + (r0 + 8 * g + (li >> 2)) * pitch + c0 + 4 * (li & 3);
  const bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0));
  const bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + 4 * pitch));
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
// An accumulator tile (rows r0 + 4g + r, column c0 + i) into a bf16 LDS tile.
__device__ __forceinline__ void put_acc(bf16* M, int pitch, int r0, int c0, int lane, f32x4 x) {
  const int g = lane >> 4, li = lane & 15;
#pragma unroll
  for (int r = 0; r < 4; ++r) M[(r0 + 4 * g + r) * pitch + c0 + li] = static_cast<bf16>(x[r]);
}
__device__ __forceinline__ bf16x4 ld4b(const bf16* p) { return *reinterpret_cast<const bf16x4*>(p); }

// ---------------------------------------------------------------- chunk -> sequence
struct ChunkLoc {
  int64_t n, c, c0;
  int len;
};
// Item = global chunk index (sequence n's chunks are chunk_first[n] + c with cu_seqlens, n * ceil(T/64) + c
// without); false for grid items past the last chunk.
__device__ __forceinline__ bool locate_chunk(const ChunkBwdParams& p, int64_t item, ChunkLoc& L) {
  int64_t bos, eos;
  if (p.cu) {
    if (item >= p.chunk_first[p.N]) return false;
    int64_t lo = 0, hi = p.N - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (p.chunk_first[mid] <= item) lo = mid;
      else hi = mid - 1;
    }
    L.n = lo;
    L.c = item - p.chunk_first[lo];
    bos = load_index(p.cu, p.cu_i32, lo);
    eos = load_index(p.cu, p.cu_i32, lo + 1);
  } else {
    const int64_t ncs = (p.T + kC - 1) / kC;
    L.n = item / ncs;
    L.c = item % ncs;
    bos = L.n * p.T;
    eos = bos + p.T;
  }
  L.c0 = bos + L.c * kC;
  L.len = (int)((eos - L.c0) < kC ? (eos - L.c0) : kC);
  return true;
}

// Staging of a chunk's tiles into LDS, split into fetch (the global loads, into registers) and put
// (the LDS writes): a caller issues every fetch of a step before the first put, so the loads are in
// flight together instead of one round trip per tile. Rows past len read as zeros (buffer range).
//
// q/k rows [64][KD] (bf16; L2-normalised and rounded to bf16 at the put when asked, exactly as the
// forward stages them); NT threads, tid < NT.
template <int KD, int NT>
struct QKRows {
  static constexpr int KCH = KD / 8, RPP = NT / KCH, N = kC / RPP;
  bf16x8 x[N];
};
template <int KD, int NT>
__device__ __forceinline__ void fetch_qk(QKRows<KD, NT>& r, const bf16* src, int64_t H, int len, int tid) {
  using R = QKRows<KD, NT>;
  const uint32_t rb = (uint32_t)(H * KD * 2);
  const auto rs = make_rsrc(src, (uint32_t)len * rb);
  const int row = tid / R::KCH, ch = tid % R::KCH;
#pragma unroll
  for (int u = 0; u < R::N; ++u) r.x[u] = buf_load16(rs, (uint32_t)(row + u * R::RPP) * rb + ch * 16);
}
template <int KD, int NT>
__device__ __forceinline__ void put_qk(const QKRows<KD, NT>& r, bf16* dst, int pitch, bool l2, int tid) {
  using R = QKRows<KD, NT>;
  const int row = tid / R::KCH, ch = tid % R::KCH;
#pragma unroll
  for (int u = 0; u < R::N; ++u)
    *reinterpret_cast<bf16x8*>(dst + (row + u * R::RPP) * pitch + ch * 8) = l2 ? l2norm_row_chunk<R::KCH>(r.x[u]) : r.x[u];
}
// A [64][W] slice (16-byte pieces) of a [tokens][heads][*] tensor with row stride rb bytes.
template <int W, int NT>
struct Slice {
  static constexpr int CH = W / 8, N = kC * CH / NT;
  static_assert(kC * CH % NT == 0, "slice pieces must divide among the threads");
  u32x4 x[N];
};
template <int W, int NT>
__device__ __forceinline__ void fetch_slice(Slice<W, NT>& r, const void* src, uint32_t rb, int len, int tid) {
  using R = Slice<W, NT>;
  const auto rs = make_rsrc(src, (uint32_t)len * rb);
#pragma unroll
  for (int u = 0; u < R::N; ++u) {
    const int e = u * NT + tid, row = e / R::CH, ch = e % R::CH;
    r.x[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)((uint32_t)row * rb + ch * 16), 0, 0);
  }
}
template <int W, int NT, typename E>
__device__ __forceinline__ void put_slice(const Slice<W, NT>& r, E* dst, int pitch, int tid) {
  using R = Slice<W, NT>;
  constexpr int EPC = 16 / sizeof(E);  // elements per 16-byte piece
#pragma unroll
  for (int u = 0; u < R::N; ++u) {
    const int e = u * NT + tid, row = e / R::CH, ch = e % R::CH;
    *reinterpret_cast<u32x4*>(dst + row * pitch + ch * EPC) = r.x[u];
  }
}
// Gate terms of a chunk (one wave, lane = token), as the forward computes them: raw loads, then the put.
__device__ __forceinline__ void fetch_gates_bwd(uint32_t& graw, uint32_t& braw, const ChunkBwdParams& p, int64_t c0,
                                                int64_t hv, int len, int lane) {
  const uint32_t gb = (uint32_t)(p.HV * dtype_bytes(p.dg)), bb = (uint32_t)(p.HV * dtype_bytes(p.db));
  const auto rg = make_rsrc(static_cast<const char*>(p.g) + (c0 * p.HV + hv) * dtype_bytes(p.dg), (uint32_t)len * gb);
  const auto rb = make_rsrc(static_cast<const char*>(p.beta) + (c0 * p.HV + hv) * dtype_bytes(p.db), (uint32_t)len * bb);
  graw = buf_load_raw32(rg, lane * gb, p.dg);
  braw = buf_load_raw32(rb, lane * bb, p.db);
}
__device__ __forceinline__ void put_gates_bwd(ChunkGates& gs, uint32_t graw, uint32_t braw, const ChunkBwdParams& p,
                                              int64_t hv, int len, int lane) {
  chunk_gates_from_raw(gs, graw, braw, p.dg, p.db, len, p.flags, p.A_log ? p.A_log[hv] : 0.f,
                       p.dt_bias ? p.dt_bias[hv] : 0.f, lane);
}

// ================================================================== 1. prep: T - I (natural) and G1
// One workgroup of 4 waves per (chunk, value head); wave w owns the 16 tokens 16w..16w+15 of every
// product it computes.
template <int KD, int VD>
__global__ __launch_bounds__(256) void gated_delta_chunk_bwd_prep_kernel(ChunkBwdParams p) {
  // Pitches (bf16 elements): 272-byte q/k/dO/F rows and 136-byte P/T rows at K = V = 128. F reuses
  // K's space and dO Q's: both are dead once P is computed. 53,504 bytes at K = V = 128: three
  // workgroups per CU.
  constexpr int KPB = KD + 8, VPB = VD + 8, TPB = kC + 4, KS = KD / 32, VT = VD / 16;
  constexpr int kTile = kC * (KPB > VPB ? KPB : VPB);
  __shared__ __align__(16) bf16 KFb[kTile], QOb[kTile];
  __shared__ __align__(16) bf16 Pb[kC * TPB], Tm[kC * TPB];
  bf16* const Kb = KFb;
  bf16* const Fb = KFb;
  bf16* const Qb = QOb;
  bf16* const dOb = QOb;
  __shared__ __align__(16) ChunkGates gs;
  ChunkLoc L;
  if (!locate_chunk(p, blockIdx.x, L)) return;
  const int64_t hv = blockIdx.y, h = hv / (p.HV / p.H);
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), g4 = lane >> 4, li = lane & 15;
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const int len = L.len;
  const int64_t c0 = L.c0;

  // every global load of the chunk in flight together, then the LDS writes
  QKRows<KD, 256> xk, xq;
  Slice<VD, 256> xo;
  Slice<kC, 256> xt;
  fetch_qk(xk, static_cast<const bf16*>(p.k) + (c0 * p.H + h) * KD, p.H, len, t);
  fetch_qk(xq, static_cast<const bf16*>(p.q) + (c0 * p.H + h) * KD, p.H, len, t);
  fetch_slice(xo, static_cast<const bf16*>(p.dout) + (c0 * p.HV + hv) * VD, (uint32_t)(p.HV * VD * 2), len, t);
  fetch_slice(xt, p.tw + (c0 * p.HV + hv) * kC, (uint32_t)(p.HV * kC * 2), len, t);
  uint32_t graw = 0, braw = 0;
  if (w == 0) fetch_gates_bwd(graw, braw, p, c0, hv, len, lane);
  put_qk(xk, Kb, KPB, l2, t);
  put_qk(xq, Qb, KPB, l2, t);
  {  // T - I: fp16 rows with tok_col columns -> bf16 natural columns in LDS
#pragma unroll
    for (int u8 = 0; u8 < Slice<kC, 256>::N; ++u8) {
      const int e = u8 * 256 + t, row = e >> 3, ch = e & 7, u = ch >> 2, gq = ch & 3;
      // columns 32u + 8gq + 4hh + r of the chunk hold tokens 32u + 16hh + 4gq + r
      const f16x8 x = __builtin_bit_cast(f16x8, xt.x[u8]);
      const bf16x4 lo = to_bf16x4((float)x[0], (float)x[1], (float)x[2], (float)x[3]);
      const bf16x4 hi = to_bf16x4((float)x[4], (float)x[5], (float)x[6], (float)x[7]);
      *reinterpret_cast<bf16x4*>(Tm + row * TPB + 32 * u + 4 * gq) = lo;
      *reinterpret_cast<bf16x4*>(Tm + row * TPB + 32 * u + 16 + 4 * gq) = hi;
    }
  }
  if (w == 0) put_gates_bwd(gs, graw, braw, p, hv, len, lane);
  __syncthreads();
  {  // (T - I)^T rows for the next two kernels: row t holds (T - I)[j][t], j = 0..63
#pragma unroll
    for (int u8 = 0; u8 < 2; ++u8) {
      const int e = u8 * 256 + t, row = e >> 3, j0 = (e & 7) * 8;
      bf16x8 x;
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = Tm[(j0 + j) * TPB + row];
      if (row < len) *reinterpret_cast<bf16x8*>(p.tnt + ((c0 + row) * p.HV + hv) * kC + j0) = x;
    }
  }

  // scale P = scale (Q K^T) o E (j <= t), rows 16w..16w+15 (this wave's Q fragments read once)
  bf16x8 qw[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qw[s] = frag_row(Qb, KPB, 16 * w, 32 * s, lane);
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    f32x4 acc = f32x4{};
    if (jt <= w) {
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = mma(qw[s], frag_row(Kb, KPB, 16 * jt, 32 * s, lane), acc);
    }
    const int j = 16 * jt + li;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tt = 16 * w + 4 * g4 + r;
      acc[r] = j <= tt ? p.scale * __expf(gs.gam[tt] - gs.gam[j]) * acc[r] : 0.f;
    }
    put_acc(Pb, TPB, 16 * w, 16 * jt, lane, acc);
  }
  __syncthreads();
  put_slice(xo, dOb, VPB, t);  // Q is dead
  __syncthreads();
  // F = (scale P)^T dO, rows (key tokens j) 16w..16w+15 (into K's space: K is dead now); this
  // wave's P^T fragments serve every value tile: read once
  f32x4 F[VT];
  bf16x8 pw[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) pw[s] = frag_col(Pb, TPB, 32 * s, 16 * w, lane);
#pragma unroll
  for (int ct = 0; ct < VT; ++ct) {
    F[ct] = f32x4{};
#pragma unroll
    for (int s = 0; s < 2; ++s)
      if (s == 1 || w <= 1) F[ct] = mma(pw[s], frag_col(dOb, VPB, 32 * s, 16 * ct, lane), F[ct]);
  }
#pragma unroll
  for (int ct = 0; ct < VT; ++ct) put_acc(Fb, VPB, 16 * w, 16 * ct, lane, F[ct]);
  __syncthreads();
  // G1 = F + (T - I)^T F  ((T - I)_{t'j} vanishes unless t' > j); the (T - I)^T fragments read once
#pragma unroll
  for (int u = 0; u < 2; ++u) pw[u] = frag_col(Tm, TPB, 32 * u, 16 * w, lane);
#pragma unroll
  for (int ct = 0; ct < VT; ++ct) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (u == 1 || w <= 1) F[ct] = mma(pw[u], frag_col(Fb, VPB, 32 * u, 16 * ct, lane), F[ct]);
    // the lane's 4 tokens of one value column are adjacent in the chunk-blocked G1: one 8-byte
    // store; every token slot of the chunk is written (zero past len)
    const int tt = 16 * w + 4 * g4;
    const bf16x4 gv = to_bf16x4(tt < len ? F[ct][0] : 0.f, tt + 1 < len ? F[ct][1] : 0.f,
                                tt + 2 < len ? F[ct][2] : 0.f, tt + 3 < len ? F[ct][3] : 0.f);
    *reinterpret_cast<bf16x4*>(p.g1 + (((int64_t)blockIdx.x * p.HV + hv) * VD + 16 * ct + li) * kC + tt) = gv;
  }
}

// ================================================================== 2. reverse state recurrence
// One workgroup of 4 waves per (sequence, value head, 32 value columns). Waves 0 and 1 each hold 16
// columns of dS [K x 16] in fp32 MFMA accumulators (tile a: keys 16a + 4g + r, column i) for the
// whole sequence; waves 2 and 3 stage the next chunk's tiles into the other LDS slot meanwhile.
template <int KD, int VD>
__global__ __launch_bounds__(256, 1) void gated_delta_chunk_bwd_state_kernel(ChunkBwdParams p) {
  constexpr int KPB = row_pitch<KD>(), KS = KD / 32, KT = KD / 16, NVB = VD / 32;
  constexpr int OP = 40;  // bf16 pitch of the dO slice
  __shared__ __align__(16) bf16 Kb[2][kC * KPB], Qb[2][kC * KPB], Tm[2][kC * kCPb], dOs[2][kC * OP];
  __shared__ __align__(16) bf16 G1s[2][32 * kCPb];  // G1 slice: [32 value columns][64 tokens]
  __shared__ __align__(16) ChunkGates gv[2];

  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), g4 = lane >> 4, li = lane & 15;
  // blockIdx b lands on XCD b % 8: XCD x takes chains x, x + 8, ..., all V/32 slices of a chain on
  // one XCD, so the K, Q and T - I tiles its slices all read come from one L2 (as in the forward)
  const int64_t chains = p.N * p.HV;
  int64_t chain;
  int vb;
  if (chains % 8 == 0) {
    const int64_t x = blockIdx.x % 8, j = blockIdx.x / 8;
    chain = 8 * (j / NVB) + x;
    vb = (int)(j % NVB);
  } else {
    chain = blockIdx.x / NVB;
    vb = (int)(blockIdx.x % NVB);
  }
  const int64_t n = chain / p.HV, hv = chain % p.HV, h = hv / (p.HV / p.H);
  int64_t bos, eos, cgb;
  const int64_t ncs = (p.T + kC - 1) / kC;
  if (p.cu) {
    bos = load_index(p.cu, p.cu_i32, n);
    eos = load_index(p.cu, p.cu_i32, n + 1);
    cgb = p.chunk_first[n];
  } else {
    bos = n * p.T;
    eos = bos + p.T;
    cgb = n * ncs;
  }
  const int nc = (int)((eos - bos + kC - 1) / kC);
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;

  // Loader waves (2, 3; tl = 0..127): a chunk's tiles are fetched into registers a step before they
  // are written to LDS, so each step hides a step of load latency.
  struct ChunkRegs {
    QKRows<KD, 128> xk, xq;
    Slice<kC, 128> xt;
    Slice<32, 128> xo;
    u32x4 xg[2];  // the G1 slice: 32 columns x 64 tokens, 4 KB contiguous in the chunk-blocked G1
    uint32_t graw, braw;
    int len;
  };
  auto fetch_chunk = [&](ChunkRegs& r, int c, int tl) {
    const int64_t c0 = bos + (int64_t)c * kC;
    r.len = (int)((eos - c0) < kC ? (eos - c0) : kC);
    fetch_qk(r.xk, static_cast<const bf16*>(p.k) + (c0 * p.H + h) * KD, p.H, r.len, tl);
    fetch_qk(r.xq, static_cast<const bf16*>(p.q) + (c0 * p.H + h) * KD, p.H, r.len, tl);
    fetch_slice(r.xt, p.tnt + (c0 * p.HV + hv) * kC, (uint32_t)(p.HV * kC * 2), r.len, tl);
    fetch_slice(r.xo, static_cast<const bf16*>(p.dout) + (c0 * p.HV + hv) * VD + vb * 32, (uint32_t)(p.HV * VD * 2),
                r.len, tl);
    const bf16* g1src = p.g1 + (((cgb + c) * p.HV + hv) * VD + vb * 32) * kC;
#pragma unroll
    for (int u = 0; u < 2; ++u) r.xg[u] = *reinterpret_cast<const u32x4*>(g1src + (u * 128 + tl) * 8);
    r.graw = r.braw = 0;
    if (w == 2) fetch_gates_bwd(r.graw, r.braw, p, c0, hv, r.len, lane);
  };
  auto put_chunk = [&](const ChunkRegs& r, int slot, int tl) {
    put_qk(r.xk, Kb[slot], KPB, l2, tl);
    put_qk(r.xq, Qb[slot], KPB, l2, tl);
    put_slice(r.xt, Tm[slot], kCPb, tl);
    put_slice(r.xo, dOs[slot], OP, tl);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = u * 128 + tl;  // column e / 8, tokens 8 (e % 8) .. + 7
      *reinterpret_cast<u32x4*>(G1s[slot] + (e >> 3) * kCPb + (e & 7) * 8) = r.xg[u];
    }
    if (w == 2) put_gates_bwd(gv[slot], r.graw, r.braw, p, hv, r.len, lane);
  };

  // Each role runs its own loop of nc steps with one barrier each (the counts match), so the
  // loaders' registers in flight are not live through the state waves' code.
  if (w < 2) {
    const int sw = w & 1, col = vb * 32 + 16 * sw + li;  // value column of this lane
    f32x4 dS[KT];
#pragma unroll
    for (int a = 0; a < KT; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dS[a][r] = p.dht ? p.dht[((n * p.HV + hv) * KD + 16 * a + 4 * g4 + r) * VD + col] : 0.f;
    __syncthreads();
    for (int i = 0; i < nc; ++i) {
      const int c = nc - 1 - i, slot = i & 1;
      const bf16* kb = Kb[slot];
      const bf16* qb = Qb[slot];
      const bf16* tm = Tm[slot];
      const ChunkGates& G = gv[slot];
      // W1 = K dS': contraction slots (g, j) hold keys 32s + 4g + j and 32s + 16 + 4g + j. Every
      // K fragment is read before the first MFMA.
      bf16x8 sb[KS], kf[KS][4];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        sb[s] = pack8(dS[2 * s], dS[2 * s + 1]);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const bf16* kr = kb + (16 * b + li) * KPB + 32 * s + 4 * g4;
          const bf16x4 k0 = ld4b(kr), k1 = ld4b(kr + 16);
          kf[s][b] = bf16x8{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x4 W[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) W[b] = f32x4{};
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int b = 0; b < 4; ++b) W[b] = mma(kf[s][b], sb[s], W[b]);
      // dS' of chunk c (the gradient of the state leaving it) from the bf16 operand just built,
      // transposed: keys 32s + 4g..+3 (tile 2s) and 32s + 16 + 4g..+3 (tile 2s + 1) of column col
      {
        bf16* dp = p.dhs + (((cgb + c) * p.HV + hv) * VD + col) * (int64_t)KD + 4 * g4;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          *reinterpret_cast<bf16x4*>(dp + 32 * s) = bf16x4{sb[s][0], sb[s][1], sb[s][2], sb[s][3]};
          *reinterpret_cast<bf16x4*>(dp + 32 * s + 16) = bf16x4{sb[s][4], sb[s][5], sb[s][6], sb[s][7]};
        }
      }
      // (T - I)^T fragments for dX: row 16b + i of the staged (T - I)^T tile at the contraction
      // slots' tokens 32u + 4g..+3 and 32u + 16 + 4g..+3
      bf16x8 tf[4][2];
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          if (u == 1 || b <= 1) {
            const bf16* tr = tm + (16 * b + li) * kCPb + 32 * u + 4 * g4;
            const bf16x4 t0 = ld4b(tr), t1 = ld4b(tr + 16);
            tf[b][u] = bf16x8{t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
          }
      // dX = G1 + Z + (T - I)^T Z, Z = r o W1 (token pairs 32u + 4g + r, 32u + 16 + 4g + r)
      f32x4 X[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const bf16x4 g1v = ld4b(G1s[slot] + (16 * sw + li) * kCPb + 16 * b + 4 * g4);  // tokens 16b + 4g..+3
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 16 * b + 4 * g4 + r;
          W[b][r] *= G.dlast[tok];
          X[b][r] = (float)g1v[r] + W[b][r];
        }
      }
      const bf16x8 zb[2] = {pack8(W[0], W[1]), pack8(W[2], W[3])};
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          if (u == 1 || b <= 1) X[b] = mma(tf[b][u], zb[u], X[b]);
      // dY = -beta a dX; scale a dO
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) X[b][r] *= -G.begam[16 * b + 4 * g4 + r];
      const bf16x8 yb[2] = {pack8(X[0], X[1]), pack8(X[2], X[3])};
      bf16x8 qa[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const bf16x4 d0 = ld4_tr(dOs[slot], OP, 32 * u, 16 * sw, lane), d1 = ld4_tr(dOs[slot], OP, 32 * u + 16, 16 * sw, lane);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          qa[u][m] = static_cast<bf16>(p.scale * G.egam[32 * u + 4 * g4 + m] * (float)d0[m]);
          qa[u][4 + m] = static_cast<bf16>(p.scale * G.egam[32 * u + 16 + 4 * g4 + m] * (float)d1[m]);
        }
      }
      // dS = e^{gam_c} dS' + K^T dY + Q^T (scale a dO), in two halves of the key tiles, each half's
      // K^T and Q^T fragments read before its MFMAs
      const float ac = G.egam[kC - 1];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        bf16x8 ktf[KT / 2][2], qtf[KT / 2][2];
#pragma unroll
        for (int aa = 0; aa < KT / 2; ++aa)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int a = hh * (KT / 2) + aa;
            const bf16x4 k0 = ld4_tr(kb, KPB, 32 * u, 16 * a, lane), k1 = ld4_tr(kb, KPB, 32 * u + 16, 16 * a, lane);
            ktf[aa][u] = bf16x8{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
            const bf16x4 q0 = ld4_tr(qb, KPB, 32 * u, 16 * a, lane), q1 = ld4_tr(qb, KPB, 32 * u + 16, 16 * a, lane);
            qtf[aa][u] = bf16x8{q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
          }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int aa = 0; aa < KT / 2; ++aa) {
          const int a = hh * (KT / 2) + aa;
          dS[a] *= ac;
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            dS[a] = mma(ktf[aa][u], yb[u], dS[a]);
            dS[a] = mma(qtf[aa][u], qa[u], dS[a]);
          }
        }
      }
      __syncthreads();
    }
    if (p.dh0) {
#pragma unroll
      for (int a = 0; a < KT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) p.dh0[((n * p.HV + hv) * KD + 16 * a + 4 * g4 + r) * VD + col] = dS[a][r];
    }
  } else {
    const int tl = t - 128;
    ChunkRegs nx;  // the next chunk's tiles, in flight across a step
    if (nc > 0) {
      fetch_chunk(nx, nc - 1, tl);
      put_chunk(nx, 0, tl);
      if (nc > 1) fetch_chunk(nx, nc - 2, tl);
    }
    __syncthreads();
    for (int i = 0; i < nc; ++i) {
      const int c = nc - 1 - i, slot = i & 1;
      if (i + 1 < nc) {
        put_chunk(nx, slot ^ 1, tl);                  // chunk c - 1, fetched a step ago
        if (i + 2 < nc) fetch_chunk(nx, c - 2, tl);  // chunk c - 2
      }
      __syncthreads();
    }
  }
}

// ================================================================== 3. per-chunk gradients
// One workgroup of 4 waves per (chunk, q/k head), looping over the value heads of the head (GVA:
// dq and dk are summed in registers) and, per value head, over 32-column passes of V. Wave w owns
// the tokens 16w..16w+15 of every product: the pass's two 16-column tiles, the c x c tiles (w, jt)
// with jt <= w, and all key tiles of dq and dk, so per-token sums stay inside a wave. 80,160 bytes
// of LDS and at most 256 VGPRs: two workgroups share a CU, so one's loads and barriers overlap the
// other's MFMAs. The row scalings of the state terms (scale e^gam of dQ_S, -beta e^gam of dY, r of
// Delta) are applied to the A fragments per lane (a lane's A row is one token).
template <int KD, int VD>
__global__ __launch_bounds__(256, 2) void gated_delta_chunk_bwd_grad_kernel(ChunkBwdParams p) {
  constexpr int KPB = KD + 8, KS = KD / 32, KT = KD / 16, NP = VD / 32;
  constexpr int XP = 48;      // bf16 pitch of the [64][32] pass tiles (96 B rows)
  constexpr int FP = KD + 4;  // fp32 pitch of the dq / dk rows at the end
  constexpr int NSP = KD / 64;  // 16-byte pieces per thread of a [32][KD] S^T tile
  constexpr int kSB = 32 * KPB, kPB = kC * XP;
  constexpr int kBig = 2 * kSB + 4 * kPB;  // bf16 elements
  static_assert(2 * kC * kCPb <= kBig && kC * FP * 2 <= kBig, "LDS reuse");
  __shared__ __align__(16) bf16 Kb[kC * KPB], Qb[kC * KPB];
  __shared__ __align__(16) bf16 big[kBig];
  __shared__ __align__(16) ChunkGates gs;
  // per-token row/column sums, one row per wave, added in wave order (deterministic, no atomics)
  __shared__ float tb_[4][kC], tg_[4][kC], red_[4][2];
  bf16* const SbT = big;             // S^T of the pass: [32 value columns][KD keys]
  bf16* const dSbT = big + kSB;      // dS'^T of the pass
  bf16* const dOb = big + 2 * kSB;   // [64 tokens][32 value columns]
  bf16* const Xb = dOb + kPB;        // V, then X, then r o K dS'
  bf16* const Db = Xb + kPB;         // Delta
  bf16* const dXb = Db + kPB;
  bf16* const cc1 = big;             // dG (after the passes)
  bf16* const cc2 = big + kC * kCPb; // dQK
  float* const fr = reinterpret_cast<float*>(big);  // dq or dk rows at the end

  ChunkLoc L;
  if (!locate_chunk(p, blockIdx.x, L)) return;
  const int64_t h = blockIdx.y, rep = p.HV / p.H;
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), g4 = lane >> 4, li = lane & 15;
  const int tok0 = 16 * w;
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const int len = L.len;
  const int64_t c0 = L.c0, cg = blockIdx.x;
  const uint32_t vrow = (uint32_t)(p.HV * VD * 2), trow = (uint32_t)(p.HV * kC * 2);

  // the first value head's gate loads go out first, in flight while K and Q are staged
  uint32_t graw = 0, braw = 0;
  if (w == 0) fetch_gates_bwd(graw, braw, p, c0, h * rep, len, lane);
  {  // K and Q rows: both tiles' loads in flight before the first LDS write
    QKRows<KD, 256> xk, xq;
    fetch_qk(xk, static_cast<const bf16*>(p.k) + (c0 * p.H + h) * KD, p.H, len, t);
    fetch_qk(xq, static_cast<const bf16*>(p.q) + (c0 * p.H + h) * KD, p.H, len, t);
    put_qk(xk, Kb, KPB, l2, t);
    put_qk(xq, Qb, KPB, l2, t);
  }

  f32x4 dqa[KT], dka[KT];
#pragma unroll
  for (int j = 0; j < KT; ++j) dqa[j] = dka[j] = f32x4{};

  // the global loads of a pass: S^T and dS'^T rows (all rows valid), dO and V [64][32] (rows past
  // len read as zeros), G1 in accumulator layout (tiles ct = 0, 1 of the pass)
  bf16x8 ps[NSP], pd[NSP];
  u32x4 po, pv;
  float g1c[8];
  auto fetch_pass = [&](int64_t hv, int ps_i, float (&g1)[8]) {
    const bf16* hsrc = p.hs + ((cg * p.HV + hv) * VD + 32 * ps_i) * (int64_t)KD;
    const bf16* dsrc = p.dhs + ((cg * p.HV + hv) * VD + 32 * ps_i) * (int64_t)KD;
#pragma unroll
    for (int u = 0; u < NSP; ++u) {
      ps[u] = ld8(hsrc + (int64_t)(u * 256 + t) * 8);
      pd[u] = ld8(dsrc + (int64_t)(u * 256 + t) * 8);
    }
    const int row = t >> 2, ch = t & 3;
    const auto ro = make_rsrc(static_cast<const bf16*>(p.dout) + (c0 * p.HV + hv) * VD + 32 * ps_i, (uint32_t)len * vrow);
    const auto rv = make_rsrc(static_cast<const bf16*>(p.v) + (c0 * p.HV + hv) * VD + 32 * ps_i, (uint32_t)len * vrow);
    po = __builtin_amdgcn_raw_buffer_load_b128(ro, (int)((uint32_t)row * vrow + ch * 16), 0, 0);
    pv = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)((uint32_t)row * vrow + ch * 16), 0, 0);
    // chunk-blocked G1: the lane's tokens tok0 + 4g..+3 of a column are one 8-byte load (zeros
    // past len, as the prep kernel writes them)
    const bf16* g1src = p.g1 + ((cg * p.HV + hv) * VD + 32 * ps_i + li) * kC + tok0 + 4 * g4;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const bf16x4 x = *reinterpret_cast<const bf16x4*>(g1src + 16 * ct * kC);
#pragma unroll
      for (int r = 0; r < 4; ++r) g1[4 * ct + r] = (float)x[r];
    }
  };

  for (int64_t rr = 0; rr < rep; ++rr) {
    const int64_t hv = h * rep + rr;
    if (w == 0 && rr > 0) fetch_gates_bwd(graw, braw, p, c0, hv, len, lane);
    if (t < kC) {
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        tb_[x][t] = 0.f;
        tg_[x][t] = 0.f;
      }
    }
    if (t < 8) red_[t >> 1][t & 1] = 0.f;
    if (w == 0) put_gates_bwd(gs, graw, braw, p, hv, len, lane);

    f32x4 dA[4], dP[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) dA[j] = dP[j] = f32x4{};
    float pb[4] = {0.f, 0.f, 0.f, 0.f}, pg[4] = {0.f, 0.f, 0.f, 0.f}, pr[4] = {0.f, 0.f, 0.f, 0.f};
    float sdot = 0.f;

#pragma unroll 1
    for (int pi = 0; pi < NP; ++pi) {
      fetch_pass(hv, pi, g1c);
      // T - I fragments of this wave's rows, (T - I) rows (Delta) and (T - I)^T rows (dX): loaded
      // with each pass (L2 hits after the first) so they are not live through the c x K products.
      // The (T - I) rows are the forward's fp16 rows: their 16-byte piece 4u + g holds the tokens
      // 32u + 4g..+3 and 32u + 16 + 4g..+3, the contraction slots that the Delta product's B
      // fragments (ld4_tr pairs 16 rows apart) use; converted to bf16 as read.
      bf16x8 tfr[2], tft[2];
      {
        const int lq = opaque_int(lane);
        const auto rw = make_rsrc(p.tw + (c0 * p.HV + hv) * kC, (uint32_t)len * trow);
        const auto rt = make_rsrc(p.tnt + (c0 * p.HV + hv) * kC, (uint32_t)len * trow);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t off = (uint32_t)(tok0 + (lq & 15)) * trow + (4 * u + (lq >> 4)) * 16;
          const f16x8 h = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)off, 0, 0));
          const bf16x4 lo = to_bf16x4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
          const bf16x4 hi = to_bf16x4((float)h[4], (float)h[5], (float)h[6], (float)h[7]);
          tfr[u] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          tft[u] = buf_load16(rt, off);
        }
      }
      __syncthreads();  // the previous pass (or value head) is done with the LDS tiles
#pragma unroll
      for (int u = 0; u < NSP; ++u) {
        const int e = u * 256 + t, row = e / (KD / 8), c8 = (e % (KD / 8)) * 8;
#pragma unroll
        for (int x = 0; x < 8; ++x) sdot += (float)ps[u][x] * (float)pd[u][x];
        *reinterpret_cast<bf16x8*>(SbT + row * KPB + c8) = ps[u];
        *reinterpret_cast<bf16x8*>(dSbT + row * KPB + c8) = pd[u];
      }
      *reinterpret_cast<u32x4*>(dOb + (t >> 2) * XP + (t & 3) * 8) = po;
      *reinterpret_cast<u32x4*>(Xb + (t >> 2) * XP + (t & 3) * 8) = pv;
      __syncthreads();
      // Y = K S, W = K dS', QS = Q S on the tiles (w, ct). (Fragment addresses derive from lane ids
      // passed through an empty asm per phase, so they are rebuilt where used instead of being
      // hoisted out of the loops into registers that stay live across them.)
      int ln = opaque_int(lane);
      f32x4 Y[2], W[2], QS[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) Y[ct] = W[ct] = QS[ct] = f32x4{};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 ak = frag_row(Kb, KPB, tok0, 32 * s, ln), aq = frag_row(Qb, KPB, tok0, 32 * s, ln);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const bf16x8 bs = frag_row(SbT, KPB, 16 * ct, 32 * s, ln);
          Y[ct] = mma(ak, bs, Y[ct]);
          QS[ct] = mma(aq, bs, QS[ct]);
          W[ct] = mma(ak, frag_row(dSbT, KPB, 16 * ct, 32 * s, ln), W[ct]);
        }
        __builtin_amdgcn_sched_barrier(0);  // one k-step's fragments live at a time
      }
      // X = beta V - beta a Y (V read from Xb, X written over it: each wave touches only its rows);
      // the a-term of dgam, scale a_t dO_t . (Q S)_t
      bf16x4 Vv[2];  // V is bf16: kept as loaded
      f32x4 Dl[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        Vv[ct] = ld4_tr(Xb, XP, tok0, 16 * ct, ln);
        const bf16x4 dd = ld4_tr(dOb, XP, tok0, 16 * ct, ln);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = tok0 + 4 * (ln >> 4) + r;
          Dl[ct][r] = gs.bet[tok] * (float)Vv[ct][r] - gs.begam[tok] * Y[ct][r];
          pg[r] += p.scale * gs.egam[tok] * (float)dd[r] * QS[ct][r];
        }
        put_acc(Xb, XP, tok0, 16 * ct, ln, Dl[ct]);
      }
      __syncthreads();
      // Delta = X + (T - I) X  ((T - I)_{tj} vanishes unless j < t)
      ln = opaque_int(lane);
#pragma unroll
      for (int u = 0; u < 2; ++u)
        if (u == 0 || w >= 2) {
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            const bf16x4 x0 = ld4_tr(Xb, XP, 32 * u, 16 * ct, ln), x1 = ld4_tr(Xb, XP, 32 * u + 16, 16 * ct, ln);
            Dl[ct] = mma(tfr[u], bf16x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]}, Dl[ct]);
          }
        }
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) put_acc(Db, XP, tok0, 16 * ct, ln, Dl[ct]);
      __syncthreads();
      // Z = r o (K dS') -> Xb; the r-term of dgam, r_t (K dS')_t . Delta_t
      ln = opaque_int(lane);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          W[ct][r] *= gs.dlast[tok0 + 4 * (ln >> 4) + r];
          pr[r] += W[ct][r] * Dl[ct][r];
        }
        put_acc(Xb, XP, tok0, 16 * ct, ln, W[ct]);
      }
      __syncthreads();
      // dX = G1 + Z + (T - I)^T Z
      ln = opaque_int(lane);
      f32x4 dX[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) dX[ct][r] = g1c[4 * ct + r] + W[ct][r];
#pragma unroll
      for (int u = 0; u < 2; ++u)
        if (u == 1 || w <= 1) {
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) dX[ct] = mma(tft[u], frag_col(Xb, XP, 32 * u, 16 * ct, ln), dX[ct]);
        }
      // dV = beta dX; row partials of dbeta and dgam
      bf16* const dvg = static_cast<bf16*>(p.dv);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int cc = 32 * pi + 16 * ct + (ln & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = tok0 + 4 * (ln >> 4) + r;
          if (tok < len) dvg[((c0 + tok) * p.HV + hv) * VD + cc] = static_cast<bf16>(gs.bet[tok] * dX[ct][r]);
          pb[r] += ((float)Vv[ct][r] - gs.egam[tok] * Y[ct][r]) * dX[ct][r];
          pg[r] -= gs.begam[tok] * dX[ct][r] * Y[ct][r];
        }
        put_acc(dXb, XP, tok0, 16 * ct, ln, dX[ct]);
      }
      __syncthreads();
      // c x c: dA' += dX Delta^T, dP' += dO Delta^T on the tiles (w, jt <= w)
      ln = opaque_int(lane);
      const bf16x8 ax = frag_row(dXb, XP, tok0, 0, ln), ao = frag_row(dOb, XP, tok0, 0, ln);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
        if (jt <= w) {
          const bf16x8 bd = frag_row(Db, XP, 16 * jt, 0, ln);
          dA[jt] = mma(ax, bd, dA[jt]);
          dP[jt] = mma(ao, bd, dP[jt]);
        }
      // c x K: dQ += (scale a dO) S^T, dK += (-beta a dX) S^T + (r Delta) dS'^T
      {
        const int rowt = tok0 + (ln & 15);  // the token of this lane's A row
        const float fo = p.scale * gs.egam[rowt], fy = -gs.begam[rowt], fd = gs.dlast[rowt];
        const bf16x8 ad = frag_row(Db, XP, tok0, 0, ln);
        bf16x8 so, sy, sd;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          so[x] = static_cast<bf16>(fo * (float)ao[x]);
          sy[x] = static_cast<bf16>(fy * (float)ax[x]);
          sd[x] = static_cast<bf16>(fd * (float)ad[x]);
        }
#pragma unroll
        for (int k4 = 0; k4 < KT; k4 += 4) {  // four key tiles' fragments read before their MFMAs
          bf16x8 bs[4], bd[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            bs[x] = frag_col(SbT, KPB, 0, 16 * (k4 + x), ln);
            bd[x] = frag_col(dSbT, KPB, 0, 16 * (k4 + x), ln);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            dqa[k4 + x] = mma(so, bs[x], dqa[k4 + x]);
            dka[k4 + x] = mma(sy, bs[x], dka[k4 + x]);
            dka[k4 + x] = mma(sd, bd[x], dka[k4 + x]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }

    // e^{gam_c} <S, dS'> and sum_t r_t (K dS')_t . Delta_t go to the chunk's last position
    sdot = wave_xor_sum(sdot, 1);
    if (lane == 0) red_[w][0] = sdot;
    __syncthreads();  // the passes are done with the LDS tiles: dG and dQK go over them
    // c x c elementwise: G = K K^T, QK = Q K^T; dA, dG, dQK; their row and column sums. The K and
    // Q fragments of this wave's rows serve every tile: read once.
    bf16x8 kown[KS], qown[KS];
    {
      const int ln = opaque_int(lane);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        kown[s] = frag_row(Kb, KPB, tok0, 32 * s, ln);
        qown[s] = frag_row(Qb, KPB, tok0, 32 * s, ln);
      }
    }
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const int ln = opaque_int(lane);
      f32x4 Gm = f32x4{}, QKm = f32x4{};
      if (jt <= w) {
        bf16x8 bk[KS];  // the tile's K fragments read before its MFMAs
#pragma unroll
        for (int s = 0; s < KS; ++s) bk[s] = frag_row(Kb, KPB, 16 * jt, 32 * s, ln);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          Gm = mma(kown[s], bk[s], Gm);
          QKm = mma(qown[s], bk[s], QKm);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      const int jj = 16 * jt + (ln & 15);
      f32x4 dG, dQK;
      float colp = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = tok0 + 4 * (ln >> 4) + r;
        const float e = jj <= tok ? __expf(gs.gam[tok] - gs.gam[jj]) : 0.f;
        const float dav = jj < tok ? -dA[jt][r] : 0.f;
        dG[r] = gs.bet[tok] * dav * e;
        dQK[r] = p.scale * dP[jt][r] * e;
        pb[r] += dav * Gm[r] * e;
        const float pair = dG[r] * Gm[r] + dQK[r] * QKm[r];
        pg[r] += pair;
        colp += pair;
      }
      put_acc(cc1, kCPb, tok0, 16 * jt, ln, dG);
      put_acc(cc2, kCPb, tok0, 16 * jt, ln, dQK);
      colp += __shfl_xor(colp, 16, kWave);
      colp += __shfl_xor(colp, 32, kWave);
      if ((ln >> 4) == 0 && jt <= w) tg_[w][jj] -= colp;
      __builtin_amdgcn_sched_barrier(0);  // one c x c tile at a time
    }
    float rsum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float b = group_sum<16>(pb[r]), gg = group_sum<16>(pg[r]), rr2 = group_sum<16>(pr[r]);
      if (li == 0) {
        const int tok = tok0 + 4 * g4 + r;
        tb_[w][tok] += b;
        tg_[w][tok] += gg - rr2;
        rsum += rr2;
      }
    }
    rsum = wave_xor_sum(rsum, 1);
    if (lane == 0) red_[w][1] = rsum;
    __syncthreads();
    // dQ += dQK K;  dK += dQK^T Q + dG K + dG^T K. The dQK and dG fragments of this wave's rows
    // (and of its columns, transposed) are the same for every key tile: read once.
    {
      const int ln = opaque_int(lane);
      bf16x8 qr[2], qc[2], gr[2], gc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        qr[u] = frag_row(cc2, kCPb, tok0, 32 * u, ln);
        qc[u] = frag_col(cc2, kCPb, 32 * u, tok0, ln);
        gr[u] = frag_row(cc1, kCPb, tok0, 32 * u, ln);
        gc[u] = frag_col(cc1, kCPb, 32 * u, tok0, ln);
      }
      // two key tiles at a time: their K and Q fragments read before their MFMAs
#pragma unroll
      for (int k2 = 0; k2 < KT; k2 += 2) {
        bf16x8 bk[2][2], bq[2][2];
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            bk[x][u] = frag_col(Kb, KPB, 32 * u, 16 * (k2 + x), ln);
            bq[x][u] = frag_col(Qb, KPB, 32 * u, 16 * (k2 + x), ln);
          }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int kt = k2 + x;
            dqa[kt] = mma(qr[u], bk[x][u], dqa[kt]);
            dka[kt] = mma(qc[u], bq[x][u], dka[kt]);
            dka[kt] = mma(gr[u], bk[x][u], dka[kt]);
            dka[kt] = mma(gc[u], bk[x][u], dka[kt]);
          }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // dg = reverse in-chunk cumsum of dgam; dbeta; the gate and sigmoid backwards
    if (w == 0) {
      const float ac = gs.egam[kC - 1];
      float dgam = ((tg_[0][lane] + tg_[1][lane]) + tg_[2][lane]) + tg_[3][lane];
      if (lane == kC - 1) {
        const float r0 = ((red_[0][0] + red_[1][0]) + red_[2][0]) + red_[3][0];
        const float r1 = ((red_[0][1] + red_[1][1]) + red_[2][1]) + red_[3][1];
        dgam += ac * r0 + r1;
      }
      const float incl = wave_inclusive_sum(dgam);
      const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), kWave - 1));
      float dgv = tot - incl + dgam;
      float dbv = ((tb_[0][lane] + tb_[1][lane]) + tb_[2][lane]) + tb_[3][lane];
      const int64_t gi = (c0 + lane) * p.HV + hv;
      float pa = 0.f, pd = 0.f;
      if (lane < len) {
        const float graw2 = load_as_f32(p.g, p.dg, gi);
        if (p.flags & GDN_FLAG_GATE_IN_KERNEL) {
          const float ea = __expf(p.A_log[hv]);
          const float gval = -ea * softplus_f32(graw2 + p.dt_bias[hv]);
          pa = dgv * gval;                                         // d/dA_log
          dgv = dgv * (-ea) * sigmoid_f32(graw2 + p.dt_bias[hv]);  // d/da, a the raw gate input
          pd = dgv;                                                // d/ddt_bias
        }
        if (p.flags & GDN_FLAG_BETA_SIGMOID) {
          const float sb = sigmoid_f32(load_as_f32(p.beta, p.db, gi));
          dbv *= sb * (1.f - sb);
        }
        store_from_f32(p.dgate, p.dg, gi, dgv);
        store_from_f32(p.dbeta, p.db, gi, dbv);
      }
      if (p.flags & GDN_FLAG_GATE_IN_KERNEL) {
        pa = wave_xor_sum(pa, 1);
        pd = wave_xor_sum(pd, 1);
        if (lane == 0) {
          p.gate_part[(cg * p.HV + hv) * 2] = pa;
          p.gate_part[(cg * p.HV + hv) * 2 + 1] = pd;
        }
      }
    }
  }

  // dq, then dk: rows through LDS, the L2-norm backward (x / max(|x|, eps)) on the raw rows, store
#pragma unroll 1
  for (int x = 0; x < 2; ++x) {
    __syncthreads();
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) fr[(tok0 + 4 * g4 + r) * FP + 16 * kt + li] = x == 0 ? dqa[kt][r] : dka[kt][r];
    __syncthreads();
    constexpr int KCH = KD / 8, RPP = 256 / KCH;
    const int row0 = t / KCH, ch = t % KCH;
    const uint32_t rb = (uint32_t)(p.H * KD * 2);
    const bf16* raw = static_cast<const bf16*>(x == 0 ? p.q : p.k) + (c0 * p.H + h) * KD;
    bf16* dst = static_cast<bf16*>(x == 0 ? p.dq : p.dk) + (c0 * p.H + h) * KD;
    const auto rs = make_rsrc(raw, (uint32_t)len * rb);
    bf16x8 xr[kC / RPP];
    if (l2) {
#pragma unroll
      for (int u = 0; u < kC / RPP; ++u) xr[u] = buf_load16(rs, (uint32_t)(row0 + u * RPP) * rb + ch * 16);
    }
#pragma unroll
    for (int u = 0; u < kC / RPP; ++u) {
      const int row = row0 + u * RPP;
      float d[8];
      const float4 d0 = *reinterpret_cast<const float4*>(fr + row * FP + ch * 8);
      const float4 d1 = *reinterpret_cast<const float4*>(fr + row * FP + ch * 8 + 4);
      d[0] = d0.x; d[1] = d0.y; d[2] = d0.z; d[3] = d0.w;
      d[4] = d1.x; d[5] = d1.y; d[6] = d1.z; d[7] = d1.w;
      if (l2) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)xr[u][e] * (float)xr[u][e];
        ss = group_sum<KCH>(ss);
        const float nrm = sqrtf(ss);
        const float inv = 1.f / fmaxf(nrm, 1e-12f);
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dot += (float)xr[u][e] * inv * d[e];
        dot = group_sum<KCH>(dot);
        if (nrm <= 1e-12f) dot = 0.f;  // clamped norm: x / eps is linear in x
#pragma unroll
        for (int e = 0; e < 8; ++e) d[e] = (d[e] - (float)xr[u][e] * inv * dot) * inv;
      }
      if (row < len) {
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = static_cast<bf16>(d[e]);
        *reinterpret_cast<bf16x8*>(dst + (int64_t)row * p.H * KD + ch * 8) = o;
      }
    }
  }
}

// ================================================================== 4. dA_log, ddt_bias per head
__global__ __launch_bounds__(256) void gated_delta_gate_param_grad_kernel(const float* part, int64_t chunks,
                                                                          const int* chunk_first, int64_t N, int64_t HV,
                                                                          float* dA_log, float* ddt_bias) {
  __shared__ float red[2][4];
  const int64_t hv = blockIdx.x;
  const int64_t nch = chunk_first ? chunk_first[N] : chunks;
  float a = 0.f, d = 0.f;
  for (int64_t c = threadIdx.x; c < nch; c += 256) {
    a += part[(c * HV + hv) * 2];
    d += part[(c * HV + hv) * 2 + 1];
  }
  a = wave_xor_sum(a, 1);
  d = wave_xor_sum(d, 1);
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = a;
    red[1][threadIdx.x >> 6] = d;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    dA_log[hv] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    ddt_bias[hv] = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  }
}

}  // namespace gdn

using namespace gdn;

namespace {

int64_t chunk_bound(int64_t B, int64_t T, int64_t N, bool varlen) {
  return varlen ? (T + kC - 1) / kC + N : B * ((T + kC - 1) / kC);
}

}  // namespace

extern "C" size_t gdn_chunk_states_size(int64_t B, int64_t T, int64_t HV, int64_t K, int64_t V, int64_t N, int varlen) {
  if (B <= 0 || T < 0 || HV <= 0 || K <= 0 || V <= 0 || N <= 0) return 0;
  return (size_t)(chunk_bound(B, T, N, varlen != 0) * HV * K * V * 2);
}

extern "C" size_t gdn_chunk_bwd_workspace_size(int64_t B, int64_t T, int64_t HV, int64_t K, int64_t V, int64_t N,
                                               int varlen) {
  if (B <= 0 || T < 0 || HV <= 0 || K <= 0 || V <= 0 || N <= 0) return 0;
  const int64_t tok = B * T, ch = chunk_bound(B, T, N, varlen != 0);
  return (size_t)(align256(tok * HV * kC * 2) + align256(ch * HV * V * kC * 2) + align256(ch * HV * K * V * 2) +
                  align256(ch * HV * 2 * 4));
}

extern "C" int gdn_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                             const void* d_o, const float* d_final_state, const void* chunk_states,
                             const void* fwd_workspace, const void* cu_seqlens, int64_t B, int64_t T, int64_t H,
                             int64_t HV, int64_t K, int64_t V, int64_t N, int qkv_dtype, int g_dtype, int beta_dtype,
                             float scale, unsigned flags, const float* A_log, const float* dt_bias, void* dq, void* dk,
                             void* dv, void* dg, void* dbeta, float* d_initial_state, float* dA_log, float* ddt_bias,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !g || !beta || !d_o || !chunk_states || !fwd_workspace || !dq || !dk || !dv || !dg || !dbeta) {
    gdn_internal_set_error("gdn_chunk_bwd: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || H <= 0 || HV <= 0 || HV % H || N <= 0 || (cu_seqlens ? B != 1 : N != B)) {
    gdn_internal_set_error("gdn_chunk_bwd: bad sizes B=%lld T=%lld H=%lld HV=%lld N=%lld", (long long)B, (long long)T,
                           (long long)H, (long long)HV, (long long)N);
    return GDN_ERR_INVALID;
  }
  if ((flags & GDN_FLAG_GATE_IN_KERNEL) && (!A_log || !dt_bias || !dA_log || !ddt_bias)) {
    gdn_internal_set_error("gdn_chunk_bwd: gate in kernel needs A_log, dt_bias and their gradient outputs");
    return GDN_ERR_INVALID;
  }
  if ((K != 64 && K != 128) || (V != 64 && V != 128) || qkv_dtype != GDN_DTYPE_BF16) {
    gdn_internal_set_error("gdn_chunk_bwd: K=%lld V=%lld dtype %d unsupported (64/128, bf16)", (long long)K, (long long)V,
                           qkv_dtype);
    return GDN_ERR_UNSUPPORTED;
  }
  const bool varlen = cu_seqlens != nullptr;
  const size_t need = gdn_chunk_bwd_workspace_size(B, T, HV, K, V, N, varlen);
  if (!workspace || workspace_bytes < need) {
    gdn_internal_set_error("gdn_chunk_bwd: workspace of %zu bytes needed (got %zu)", need, workspace ? workspace_bytes : (size_t)0);
    return GDN_ERR_INVALID;
  }
  if (T == 0) return GDN_OK;
  const int64_t tok = B * T, chunks = chunk_bound(B, T, N, varlen);
  if (chunks > 0x7fffffff || HV > 65535 || N * HV * (V / 32) > 0x7fffffff) {
    gdn_internal_set_error("gdn_chunk_bwd: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  char* ws = static_cast<char*>(workspace);
  const char* fws = static_cast<const char*>(fwd_workspace);
  ChunkBwdParams p{};
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta; p.dout = d_o;
  p.dht = d_final_state;
  p.hs = static_cast<const bf16*>(chunk_states);
  p.tw = reinterpret_cast<const f16*>(fws);
  const int64_t tnb = align256(tok * HV * kC * 2);
  p.tnt = reinterpret_cast<bf16*>(ws);
  const int64_t g1b = align256(chunks * HV * V * kC * 2);
  p.g1 = reinterpret_cast<bf16*>(ws + tnb);
  p.dhs = reinterpret_cast<bf16*>(ws + tnb + g1b);
  p.gate_part = reinterpret_cast<float*>(ws + tnb + g1b + align256(chunks * HV * K * V * 2));
  p.cu = cu_seqlens;
  p.chunk_first = varlen ? reinterpret_cast<const int*>(fws + chunk_t_bytes(tok, HV)) : nullptr;
  p.cu_i32 = (flags & GDN_FLAG_CU_INT32) ? 1 : 0;
  p.T = T; p.H = H; p.HV = HV; p.N = N;
  p.dg = g_dtype; p.db = beta_dtype;
  p.scale = scale; p.flags = flags;
  p.A_log = A_log; p.dt_bias = dt_bias;
  p.dq = dq; p.dk = dk; p.dv = dv; p.dgate = dg; p.dbeta = dbeta;
  p.dh0 = d_initial_state; p.dA_log = dA_log; p.ddt_bias = ddt_bias;
  hipStream_t s = static_cast<hipStream_t>(stream);

#define GDN_BWD_DISPATCH(KERNEL, GRID, BLOCK)                                                          \
  do {                                                                                                 \
    if (K == 128 && V == 128) hipLaunchKernelGGL((KERNEL<128, 128>), GRID, BLOCK, 0, s, p);           \
    else if (K == 64 && V == 64) hipLaunchKernelGGL((KERNEL<64, 64>), GRID, BLOCK, 0, s, p);          \
    else if (K == 128 && V == 64) hipLaunchKernelGGL((KERNEL<128, 64>), GRID, BLOCK, 0, s, p);        \
    else hipLaunchKernelGGL((KERNEL<64, 128>), GRID, BLOCK, 0, s, p);                                  \
  } while (0)
  GDN_BWD_DISPATCH(gated_delta_chunk_bwd_prep_kernel, dim3((unsigned)chunks, (unsigned)HV), dim3(256));
  int rc = gdn_internal_check_launch("gated_delta_chunk_bwd_prep_kernel");
  if (rc != GDN_OK) return rc;
  GDN_BWD_DISPATCH(gated_delta_chunk_bwd_state_kernel, dim3((unsigned)(N * HV * (V / 32))), dim3(256));
  rc = gdn_internal_check_launch("gated_delta_chunk_bwd_state_kernel");
  if (rc != GDN_OK) return rc;
  GDN_BWD_DISPATCH(gated_delta_chunk_bwd_grad_kernel, dim3((unsigned)chunks, (unsigned)H), dim3(256));
  rc = gdn_internal_check_launch("gated_delta_chunk_bwd_grad_kernel");
  if (rc != GDN_OK) return rc;
#undef GDN_BWD_DISPATCH
  if (flags & GDN_FLAG_GATE_IN_KERNEL) {
    hipLaunchKernelGGL(gated_delta_gate_param_grad_kernel, dim3((unsigned)HV), dim3(256), 0, s, p.gate_part, chunks,
                       p.chunk_first, N, HV, dA_log, ddt_bias);
    rc = gdn_internal_check_launch("gated_delta_gate_param_grad_kernel");
  }
  return rc;
}
