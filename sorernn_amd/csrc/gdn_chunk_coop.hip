// The cooperative chunked prefill of the gated delta rule (inference, K = V = 128) for gfx950: one
// launch, no T-solve kernel before it and no per-chunk matrices through HBM.
//
// Per chunk of c <= 64 tokens with gam = in-chunk cumsum of g (sore/model/gdn_ref.py:17-21 in chunk
// form, restated in oracle/gdn_oracle.py::_chunk_segment), and the chunk's 16-token blocks r, c:
//   A_tj = beta_t exp(gam_t - gam_j) k_t.k_j (j < t)            T_rr = (I + A_rr)^-1 (diagonal blocks)
//   X    = diag(beta) V - diag(beta exp(gam)) K S
//   Delta_r = b_r + (T_rr - I) b_r,  b_r = X_r - sum_{c<r} A_rc Delta_c   (block forward substitution
//             of (I + A) Delta = X: no inverse of the whole 64 x 64 system is ever formed)
//   O    = scale (diag(exp(gam)) Q S + P Delta),  P_tj = exp(gam_t - gam_j) q_t.k_j (j <= t)
//   S'   = exp(gam_c) S + K^T diag(exp(gam_c - gam)) Delta
//
// Work split. One workgroup of 8 waves per (sequence, value head, 32-column slice of V); the four
// slices of a (sequence, head) chain run on one XCD (blockIdx b runs on XCD b % 8) and share its L2.
//   Waves 0, 1 (SIMDs 0, 1) -- the chain: Y = K S, X, the block substitution, the state update, for
//     16 state columns each, S [K x 16] in fp32 MFMA accumulators for the whole sequence. They
//     publish S (fp16) and Delta (fp16) of every chunk to LDS.
//   Waves 2, 3 (SIMDs 2, 3) -- the output: Z = S^T Q^T and O = scale(e^gam Z + P Delta) of the same
//     columns, one step behind the chain.
//   Waves 6, 7 (SIMDs 2, 3) -- q/k staging: the next chunk's rows (L2-normalised when asked) in fp16.
//   Wave 4 (SIMD 0) -- copies the next chunk's package and V slice into LDS (buffer_load ... lds).
//   Wave 5 (SIMD 1) -- stores O to HBM.
// The state-independent matrices of a chunk -- P, the A blocks below the diagonal, T_rr - I and the
// gate terms: its "package" -- are the same for the four slices. Slice (chunk % 4) computes it, four
// steps ahead, on waves 2, 3, 6 and 7, into a ring of packages in L2 (the workspace), and raises
// one flag per producing wave; every slice copies the package into its LDS a step before its chain
// needs it and then acknowledges it, and a producer waits for the acknowledgements before it
// reuses a ring slot. Each slice thus does a quarter of the Gram, P and T work of the chain.
//
// Coherence. Within an XCD the L2 is the coherence point: the producer's plain stores reach it
// before its flag store (s_waitcnt vmcnt(0) between them), and consumers read flags and packages
// with device-scope (sc1) loads, which miss in the CU's L1. The four slices check at start-up,
// through write-through (sc1) stores, that they share an XCD; if not, the producers write with sc1
// stores (write-through to memory), which the consumers' sc1 loads see from any XCD. Every wait is
// bounded; a wait that runs out sets the error word and the range flag and the kernel completes.
//
// Precision: as the two-kernel prefill -- fp16 MFMA operands (S, X, Delta, T_rr - I, A, P) with fp32
// accumulation, bf16 q/k products exact; the block substitution keeps b_r in the fp32 accumulator
// and rounds only the (T_rr - I) b_r operand (a CPU simulation at config-1 statistics: final-state
// relative L2 2.19e-4, as with the full inverse).

#include <algorithm>
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

namespace {

constexpr int kCoopNT = 512;
constexpr int kVBc = 32;     // value columns per workgroup
constexpr int kRing = 8;     // packages in flight per chain
constexpr int kLead = 5;     // a package is started kLead steps before its chunk
// package image in a ring slot (bytes): P rows, the 10 T/A blocks, the gate terms
constexpr int kPkgP = 0, kPkgTA = 8192, kPkgG = 8192 + 5120, kSlotBytes = 16384;
constexpr int kSyncWords = 8;  // per (chain, slot): flags of the four producing waves, acks of the four slices
constexpr int kHeadWords = 8;  // per chain: XCC ids of the four slices (+1), posted at start-up
constexpr unsigned kSpinMax = 1u << 21;

typedef __attribute__((address_space(3))) void lds_void;

// TA block index: diagonal r -> r (holds T_rr - I); below the diagonal (r, c) -> 4 + r(r-1)/2 + c
// (holds -A_rc). Each block is 16 x 16 fp16, row-major 32-byte rows; the 8-byte piece q of row i
// sits at piece q ^ (i >> 3) (no bank conflict between rows i and i + 8 in the chain's reads).
__device__ __forceinline__ constexpr int ta_blk(int r, int c) { return r == c ? r : 4 + r * (r - 1) / 2 + c; }
__device__ __forceinline__ constexpr int ta_off(int i, int q) { return i * 16 + ((q ^ (i >> 3)) << 2); }  // f16 elements

__device__ __forceinline__ f32x4 mma16h(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x4 pack4h(f32x4 a) { return to_f16x4(a[0], a[1], a[2], a[3]); }

__device__ __forceinline__ unsigned xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20); }

// Cache policy bits of the buffer instructions (gfx950): sc1 = device scope.
constexpr int kSC1 = 16;

__device__ __forceinline__ unsigned ld_sync(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kSC1);
}
__device__ __forceinline__ void st_sync(unsigned v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, (int)off, 0, kSC1);
}

}  // namespace

struct CoopParams {
  const void *q, *k, *v, *g, *beta;
  const float* h0;
  void* o;
  float* ht;
  const void* cu;
  const int* order;  // with cu: sequences by length, longest first
  int cu_i32;
  int64_t T, H, HV, N;
  int dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
  char* ring;          // [chains][ring_slots][kSlotBytes]
  int ring_slots;      // min(kRing, chunks of the longest possible sequence)
  unsigned* sync;      // [chains][kHeadWords + kRing * kSyncWords], zero on entry
  unsigned* range_flag;
  unsigned* err;       // set to 1 when a wait runs out (never expected)
};

template <int KD, int VD>
__global__ __launch_bounds__(kCoopNT, 1) void gated_delta_chunk_coop_kernel(CoopParams p) {
  static_assert(KD == 128 && VD == 128, "the cooperative prefill is built for K = V = 128");
  constexpr int NVB = VD / kVBc;  // 4 slices per chain
  constexpr int KP = KD;          // q/k rows unpadded, 16-byte chunk c of row r at c ^ ((r & 7) << 1)
  constexpr int KS = KD / 32;     // 4 MFMA k-steps over the key dim
  constexpr int KT = KD / 16;     // 8 state tiles
  constexpr int KCH = KD / 8;     // 16-byte chunks per row

  __shared__ __align__(16) f16 Kc[2][kC * KP];       // K of chunk c in slot c % 2 (fp16)
  __shared__ __align__(16) f16 Qc[2][kC * KP];       // Q of chunk c in slot c % 2 (fp16)
  __shared__ __align__(16) f16 TAc[2][10 * 256];     // T_rr - I and -A_rc of chunk c in slot c % 2
  __shared__ __align__(16) f16 Pc[2][kC * kC];       // scale * P of chunk c in slot c % 2 (tok_col, tp_off)
  __shared__ __align__(16) ChunkGates Gc[3];         // gate terms of chunk c in slot c % 3
  __shared__ __align__(16) bf16 Vc[2][kC * kVBc];    // V slice of chunk c in slot c % 2 (vo_off)
  __shared__ __align__(16) bf16 Ob[2][kC * kVBc];    // O of chunk c in slot c % 2 (vo_off)
  __shared__ __align__(16) f16x8 Sx[2][2][KS * 64];  // S entering chunk c (fp16 pairs) of chain wave w, slot c % 2
  __shared__ __align__(16) f16x8 Dx[2][2][2 * 64];   // Delta of chunk c (fp16 pairs) of chain wave w, slot c % 2
  __shared__ __align__(16) float Adiag[2][2][256];   // producer: A_rr (fp32, column-major) of the waves' two blocks
  __shared__ __align__(16) f16 Tt[2][2][256];        // producer: T_rr - I (fp16, row-major) before its store
  __shared__ __align__(16) float Gw[4][2][kC];       // producer waves' own gam / beta of the package chunk

  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), g4 = lane >> 4, li = lane & 15;

  auto kq_sw = [](int r) { return (r & 7) << 1; };
  auto kq_col = [&](int s, int l_i, int l_g) { return (((4 * s + l_g) ^ kq_sw(l_i)) << 3); };
  auto tp_off = [](int r, int col) { return r * kC + ((((col >> 3) ^ (r & 7)) << 3) | (col & 7)); };
  auto vo_off = [](int r, int col) { return r * kVBc + ((((col >> 3) ^ ((r >> 2) & 3)) << 3) | (col & 7)); };
  auto kt_pair = [&](const f16* tile, int u, int a) {  // the K^T A operand of state tile a against token pair u
    const int m = li >> 2, q = li & 3;
    const int row = 32 * u + 4 * g4 + m;
    const f16* p0 = tile + row * KP + ((((4 * (a >> 1) + q) ^ kq_sw(4 * g4 + m)) << 3) + 4 * (a & 1));
    const bf16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0));
    const bf16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + 16 * KP));
    return __builtin_bit_cast(f16x8, bf16x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]});
  };

  // ------------------------------------------------------------------ workgroup -> (chain, slice)
  // blockIdx b runs on XCD b % 8; chain 8m + x takes the blocks 32m + 8vb + x (vb = 0..3), all on XCD x.
  // Blocks of chains past the last one exit at once.
  const int64_t chains = p.N * p.HV;
  const int64_t bx = blockIdx.x, xr = bx % 8, jj = bx / 8;
  const int64_t k_rank = 8 * (jj / NVB) + xr;
  const int vb = (int)(jj % NVB);
  if (k_rank >= chains) return;
  const int hv = (int)(k_rank % p.HV);
  const int64_t n = p.order ? (int64_t)p.order[k_rank / p.HV] : k_rank / p.HV;
  const int h = hv / (int)(p.HV / p.H);
  int64_t bos, eos;
  if (p.cu) {
    bos = load_index(p.cu, p.cu_i32, n);
    eos = load_index(p.cu, p.cu_i32, n + 1);
  } else {
    bos = n * p.T;
    eos = bos + p.T;
  }
  const int nc = (int)((eos - bos + kC - 1) / kC);
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const bf16* __restrict__ qg = static_cast<const bf16*>(p.q);
  const bf16* __restrict__ kg = static_cast<const bf16*>(p.k);
  const bf16* __restrict__ vg = static_cast<const bf16*>(p.v);
  bf16* __restrict__ og = static_cast<bf16*>(p.o);
  auto chunk_len = [&](int c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    return (c >= 0 && c < nc) ? (int)((eos - c0) < kC ? (eos - c0) : kC) : 0;
  };
  const uint32_t qk_row = (uint32_t)(p.H * KD * 2), v_row = (uint32_t)(p.HV * VD * 2);

  // ring and sync words of the chain (the rank k_rank indexes them: one set per chain)
  const int R = p.ring_slots;
  char* const ring = p.ring + k_rank * (int64_t)R * kSlotBytes;
  unsigned* const syncw = p.sync + k_rank * (int64_t)(kHeadWords + kRing * kSyncWords);
  const auto rsync = make_rsrc(syncw, (uint32_t)((kHeadWords + kRing * kSyncWords) * 4));
  auto flag_off = [](int slot, int fw) { return (uint32_t)((kHeadWords + slot * kSyncWords + fw) * 4); };
  auto ack_off = [](int slot, int s) { return (uint32_t)((kHeadWords + slot * kSyncWords + 4 + s) * 4); };

  // Bounded wait until the sync word at `off` reaches `want` (device-scope loads). `dead` (uniform)
  // short-cuts every later wait once one has run out.
  auto wait_word = [&](uint32_t off, unsigned want, bool& dead) {
    if (dead) return;
    unsigned spins = 0;
    while (true) {
      const unsigned v = __builtin_amdgcn_readfirstlane(ld_sync(rsync, off));
      if ((int)(v - want) >= 0) break;
      if (++spins >= kSpinMax) {
        dead = true;
        if (lane == 0) {
          __hip_atomic_store(p.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          if (p.range_flag) __hip_atomic_store(p.range_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  };

  // ------------------------------------------------------------------ start-up
  // Post this slice's XCC id (write-through); the producing waves read all four before their first
  // ring store to choose plain (one XCD) or write-through stores.
  if (t == 0) st_sync(xcc_id() + 1, rsync, (uint32_t)(vb * 4));
  // V slots: rows past a sequence's end are never written by the copies (out-of-range lanes of
  // buffer_load ... lds leave LDS as it was), so they start as zeros and later hold earlier, finite rows.
  for (int e = t; e < 2 * kC * kVBc / 8; e += kCoopNT) reinterpret_cast<bf16x8*>(&Vc[0][0])[e] = bf16x8{};
  __syncthreads();

  const int i_begin = -kLead, i_end = nc + 2;  // every role runs these steps, one barrier each

  if (w < 2) {
    // ================================================================== chain waves
    const int sw = w;
    const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD + vb * kVBc + 16 * sw;
    f32x4 S[KT], SB[KS];
    auto sb = [&](int s) { return __builtin_bit_cast(f16x8, SB[s]); };
    auto make_sb = [&]() {
#pragma unroll
      for (int s = 0; s < KS; ++s) SB[s] = __builtin_bit_cast(f32x4, pack8h(S[2 * s], S[2 * s + 1]));
    };
    auto publish_s = [&](int slot) {
#pragma unroll
      for (int s = 0; s < KS; ++s) Sx[slot][sw][s * 64 + lane] = sb(s);
    };
    for (int i = i_begin; i < i_end; ++i) {
      if (i == -1) {
        // S (state tile a = 2s + hh: row 4g + r is key 32s + 8g + 4hh + r) from h0
#pragma unroll
        for (int a = 0; a < KT; ++a) {
          const int kd0 = 32 * (a >> 1) + 8 * g4 + 4 * (a & 1);
#pragma unroll
          for (int r = 0; r < 4; ++r) S[a][r] = p.h0 ? p.h0[sbase + (int64_t)(kd0 + r) * VD + li] : 0.f;
        }
        make_sb();
        publish_s(0);
      } else if (i >= 0 && i < nc) {
        const int ks = i & 1;
        const f16* kb = Kc[ks];
        const f16* ta = TAc[ks];
        const bf16* vp = Vc[ks];
        const ChunkGates& G = Gc[i % 3];
        // ---- Y = K S (S in fp16 pairs), with the reads for X
        f32x4 D[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) D[b] = f32x4{};
        f16x8 kf[KS][4];
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int b = 0; b < 4; ++b) kf[s][b] = ld8h(kb + (16 * b + li) * KP + kq_col(s, li, g4));
        bf16x4 vv[4];
        float4 bt[4], bg[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          vv[b] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
              (lds_bf16x4*)(vp + vo_off(16 * b + 4 * g4 + (li >> 2), 16 * sw + 4 * (li & 3))));
          bt[b] = ld4f(&G.bet[16 * b + 4 * g4]);
          bg[b] = ld4f(&G.begam[16 * b + 4 * g4]);
        }
        const float ec = __expf(G.gam[kC - 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int b = 0; b < 4; ++b) D[b] = mmah(kf[s][b], sb(s), D[b]);
        // the T / A blocks of the substitution
        f16x4 tb[10];
#pragma unroll
        for (int x = 0; x < 10; ++x) tb[x] = *reinterpret_cast<const f16x4*>(ta + x * 256 + ta_off(li, g4));
#pragma unroll
        for (int a = 0; a < KT; ++a) S[a] *= ec;
        __builtin_amdgcn_sched_barrier(0);
        // ---- X = beta V - beta e^gam Y (fp32, in the Delta accumulators)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          D[b][0] = bt[b].x * (float)vv[b][0] - bg[b].x * D[b][0];
          D[b][1] = bt[b].y * (float)vv[b][1] - bg[b].y * D[b][1];
          D[b][2] = bt[b].z * (float)vv[b][2] - bg[b].z * D[b][2];
          D[b][3] = bt[b].w * (float)vv[b][3] - bg[b].w * D[b][3];
        }
        // ---- block substitution: D_r = b_r + (T_rr - I) b_r, b_r = X_r - sum_{c<r} A_rc D_c
        D[0] = mma16h(tb[ta_blk(0, 0)], pack4h(D[0]), D[0]);
        f16x4 d0 = pack4h(D[0]);
        D[1] = mma16h(tb[ta_blk(1, 0)], d0, D[1]);
        D[2] = mma16h(tb[ta_blk(2, 0)], d0, D[2]);
        D[3] = mma16h(tb[ta_blk(3, 0)], d0, D[3]);
        D[1] = mma16h(tb[ta_blk(1, 1)], pack4h(D[1]), D[1]);
        f16x4 d1 = pack4h(D[1]);
        D[2] = mma16h(tb[ta_blk(2, 1)], d1, D[2]);
        D[3] = mma16h(tb[ta_blk(3, 1)], d1, D[3]);
        D[2] = mma16h(tb[ta_blk(2, 2)], pack4h(D[2]), D[2]);
        D[3] = mma16h(tb[ta_blk(3, 2)], pack4h(D[2]), D[3]);
        D[3] = mma16h(tb[ta_blk(3, 3)], pack4h(D[3]), D[3]);
        // ---- Delta pairs for the output waves; Delta~ = e^{gam_c - gam} Delta; K^T reads
        const f16x8 db0 = pack8h(D[0], D[1]), db1 = pack8h(D[2], D[3]);
        Dx[ks][sw][lane] = db0;
        Dx[ks][sw][64 + lane] = db1;
        f16x8 dt[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float4 dla = ld4f(&G.dlast[32 * u + 4 * g4]), dlb = ld4f(&G.dlast[32 * u + 16 + 4 * g4]);
          const f32x4 x0 = {dla.x * D[2 * u][0], dla.y * D[2 * u][1], dla.z * D[2 * u][2], dla.w * D[2 * u][3]};
          const f32x4 x1 = {dlb.x * D[2 * u + 1][0], dlb.y * D[2 * u + 1][1], dlb.z * D[2 * u + 1][2],
                            dlb.w * D[2 * u + 1][3]};
          dt[u] = pack8h(x0, x1);
        }
        f16x8 ktf[KT][2];
#pragma unroll
        for (int a = 0; a < KT; ++a)
#pragma unroll
          for (int u = 0; u < 2; ++u) ktf[a][u] = kt_pair(kb, u, a);
        __builtin_amdgcn_sched_barrier(0);
        // ---- S' = e^{gam_c} S + K^T Delta~, S' in fp16 for the next Y and for the output waves
#pragma unroll
        for (int a = 0; a < KT; ++a)
#pragma unroll
          for (int u = 0; u < 2; ++u) S[a] = mmah(ktf[a][u], dt[u], S[a]);
        make_sb();
        publish_s((i + 1) & 1);
      }
      __syncthreads();
    }
    if (p.ht) {
      uint32_t smax = 0;
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kd0 = 32 * (a >> 1) + 8 * g4 + 4 * (a & 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p.ht[sbase + (int64_t)(kd0 + r) * VD + li] = S[a][r];
          smax = max(smax, __float_as_uint(S[a][r]) & 0x7fffffffu);
        }
      }
      if (p.range_flag && smax >= 0x7f800000u)
        __hip_atomic_store(p.range_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return;
  }

  // ------------------------------------------------------------------ package production
  // Producing waves 2, 3, 6, 7 (index pw = 0..3) each own a set of 16 x 16 tiles (rt, ct), rt >= ct,
  // of the chunk's P and A:
  //   pw 0 (wave 2): (0,0) (3,0) (3,3)   -- and the diagonal solves of blocks 0 and 3
  //   pw 1 (wave 3): (1,1) (2,1) (2,2)   -- and the diagonal solves of blocks 1 and 2
  //   pw 2 (wave 6): (1,0) (2,0)         -- and the gate terms of the package
  //   pw 3 (wave 7): (3,1) (3,2)         -- and the zero tiles of P above the diagonal
  // Phase A (step j - 5): loads of the q/k fragments and raw gates of chunk j into registers.
  // Phase B (step j - 4): gates, Gram and P tiles, stores of P, -A_rc and (pw 2) the gate terms;
  //   A_rr of the diagonal tiles to LDS. Waves 6 and 7 raise their flag here.
  // Phase C (step j - 3): waves 2 and 3 solve their diagonal blocks, store T_rr - I, raise their flag.
  // A ring slot is reused kRing chunks later, once all four slices have acknowledged it.
  const int pw = (w == 2) ? 0 : (w == 3) ? 1 : (w == 6) ? 2 : 3;
  // the tiles of producing wave pw, as compile-time lists inside produce_b
  bool dead = false;
  bool wt = false;  // write-through ring stores (set when the chain's slices are not on one XCD)
  bool wt_known = false;
  auto decide_wt = [&]() {
    if (wt_known) return;
#pragma unroll
    for (int s = 0; s < NVB; ++s) wait_word((uint32_t)(s * 4), 1u, dead);
    unsigned id0 = __builtin_amdgcn_readfirstlane(ld_sync(rsync, 0));
    bool same = true;
#pragma unroll
    for (int s = 1; s < NVB; ++s) same = same && (__builtin_amdgcn_readfirstlane(ld_sync(rsync, (uint32_t)(s * 4))) == id0);
    wt = !same;
    wt_known = true;
  };
  auto ring_rsrc = [&](int j) { return make_rsrc(ring + (int64_t)(j % R) * kSlotBytes, (uint32_t)kSlotBytes); };
  auto st8 = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, f16x4 v) {
    const u32x2 x = __builtin_bit_cast(u32x2, v);
    if (wt) __builtin_amdgcn_raw_buffer_store_b64(x, r, (int)off, 0, kSC1);
    else __builtin_amdgcn_raw_buffer_store_b64(x, r, (int)off, 0, 0);
  };
  auto st4 = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    if (wt) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, kSC1);
    else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, 0);
  };
  auto raise_flag = [&](int j) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the package stores are in L2 (or memory)
    if (lane == 0) {
      if (wt) __builtin_amdgcn_raw_buffer_store_b32((unsigned)(j + 1), rsync, (int)flag_off(j % R, pw), 0, kSC1);
      else __builtin_amdgcn_raw_buffer_store_b32((unsigned)(j + 1), rsync, (int)flag_off(j % R, pw), 0, 0);
    }
  };

  // Fragment loads of a package chunk (phase A): K and Q row tiles, lane (g, i) holds row 16 tt + i,
  // keys 32 s + 8 g .. + 7 (bf16, the q/k tensors as given); rows past the chunk read as zeros.
  auto frag_rsrc = [&](const bf16* src, int c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    return make_rsrc(src + (c0 * p.H + h) * KD, (uint32_t)chunk_len(c) * qk_row);
  };
  auto load_tile = [&](bf16x8 (&dst)[KS], __amdgpu_buffer_rsrc_t r, int tt) {
    const uint32_t base = (uint32_t)(16 * tt + li) * qk_row + (uint32_t)(8 * g4) * 2;
#pragma unroll
    for (int s = 0; s < KS; ++s) dst[s] = buf_load16(r, base + (uint32_t)(64 * s));
  };
  // L2 norm of the rows of a fragment tile: a row's 128 keys are the lane's 4 fragments and those of
  // lanes i + 16, i + 32, i + 48; fp32 sums, 1 / max(||x||, 1e-12) as rsq, rounded to bf16.
  auto norm_tile = [&](bf16x8 (&x)[KS]) {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)x[s][e] * (float)x[s][e];
    ss += __shfl_xor(ss, 16, kWave);
    ss += __shfl_xor(ss, 32, kWave);
    const float inv = __builtin_amdgcn_rsqf(fmaxf(ss, 1e-24f));
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[s][e] = static_cast<bf16>((float)x[s][e] * inv);
  };
  // raw gate bits of chunk c for lane = token (a 32-bit and a 16-bit load per tensor through
  // resources sized to the dtype actually used; see the two-kernel prefill for the reason)
  struct GateBits {
    uint32_t g32, g16, b32, b16;
  };
  auto fetch_gates = [&](int c, GateBits& r) {
    const int64_t c0 = bos + (int64_t)c * kC;
    const uint32_t eg = (uint32_t)dtype_bytes(p.dg), eb = (uint32_t)dtype_bytes(p.db);
    const uint32_t gb = (uint32_t)p.HV * eg, bb = (uint32_t)p.HV * eb;
    const uint32_t len = (uint32_t)chunk_len(c);
    const uint32_t gext = len ? (len - 1) * gb + eg : 0u, bext = len ? (len - 1) * bb + eb : 0u;
    const char* gsrc = static_cast<const char*>(p.g) + (c0 * p.HV + hv) * eg;
    const char* bsrc = static_cast<const char*>(p.beta) + (c0 * p.HV + hv) * eb;
    const auto rg32 = make_rsrc(gsrc, eg == 4 ? gext : 0u), rg16 = make_rsrc(gsrc, eg == 4 ? 0u : gext);
    const auto rb32 = make_rsrc(bsrc, eb == 4 ? bext : 0u), rb16 = make_rsrc(bsrc, eb == 4 ? 0u : bext);
    r.g32 = __builtin_amdgcn_raw_buffer_load_b32(rg32, (int)(lane * gb), 0, 0);
    r.g16 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rg16, (int)(lane * gb), 0, 0);
    r.b32 = __builtin_amdgcn_raw_buffer_load_b32(rb32, (int)(lane * bb), 0, 0);
    r.b16 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb16, (int)(lane * bb), 0, 0);
  };
  const float a_log = p.A_log ? p.A_log[hv] : 0.f, dt_b = p.dt_bias ? p.dt_bias[hv] : 0.f;
  // gate terms of chunk c for lane = token: gam, e^gam, beta, beta e^gam, e^{gam_c - gam}
  auto gate_terms = [&](int c, const GateBits& r, float (&gt)[5]) {
    const uint32_t graw = p.dg == GDN_DTYPE_F32 ? r.g32 : r.g16, braw = p.db == GDN_DTYPE_F32 ? r.b32 : r.b16;
    float gval = raw32_to_f32(graw, p.dg), bval = raw32_to_f32(braw, p.db);
    if (lane < chunk_len(c)) {
      constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.6931471805599453f;
      if (p.flags & GDN_FLAG_GATE_IN_KERNEL) {
        const float x = gval + dt_b;
        const float sp = x > 20.f ? x : __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(x * kLog2e)) * kLn2;
        gval = -__builtin_amdgcn_exp2f(a_log * kLog2e) * sp;
      }
      if (p.flags & GDN_FLAG_BETA_SIGMOID) bval = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-bval * kLog2e));
    } else {
      gval = 0.f;
      bval = 0.f;
    }
    const float cs = wave_inclusive_sum(gval);
    const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cs), kWave - 1));
    const float e = __expf(cs);
    gt[0] = cs;
    gt[1] = e;
    gt[2] = bval;
    gt[3] = bval * e;
    gt[4] = __expf(last - cs);
  };

  // One tile (rt, ct) of P and of the Gram matrix from fragment tiles: kA = K rows of tile ct (A
  // operand), qB / kB = Q and K rows of tile rt (B operands). The accumulator lane (g, i) holds
  // token t = 16 rt + i against j = 16 ct + 4 g + r. Stores scale * P into the ring's P image
  // (row t, tok_col columns, tp_off) and -A into TA block (rt, ct) (ct < rt) or A_rr into LDS (fp32,
  // column-major) for the diagonal solve.
  auto pg_tile = [&](int rt, int ct, const bf16x8 (&kA)[KS], const bf16x8 (&qB)[KS], const bf16x8 (&kB)[KS],
                     __amdgpu_buffer_rsrc_t rr, float* adiag) {
    f32x4 ap{}, ag{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      ap = mma(kA[s], qB[s], ap);
      ag = mma(kA[s], kB[s], ag);
    }
    const float* gam = Gw[pw][0];
    const float* bet = Gw[pw][1];
    const int tt = 16 * rt + li, j0 = 16 * ct + 4 * g4;
    const float gt = gam[tt], bt_ = bet[tt];
    const float4 gj = ld4f(&gam[j0]);
    const float gjv[4] = {gj.x, gj.y, gj.z, gj.w};
    float pv[4], av[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool le = ct < rt || j0 + r <= tt, lt = ct < rt || j0 + r < tt;
      const float e = le ? __expf(gt - gjv[r]) : 0.f;
      pv[r] = p.scale * e * ap[r];
      av[r] = lt ? bt_ * e * ag[r] : 0.f;
    }
    st8(rr, (uint32_t)(kPkgP + tp_off(tt, tok_col(j0)) * 2), to_f16x4(pv[0], pv[1], pv[2], pv[3]));
    if (ct < rt) {
      st8(rr, (uint32_t)(kPkgTA + (ta_blk(rt, ct) * 256 + ta_off(li, g4)) * 2),
          to_f16x4(-av[0], -av[1], -av[2], -av[3]));
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) adiag[(4 * g4 + r) * 16 + li] = av[r];  // column j, row t
    }
  };

  // The diagonal solves of a wave's two blocks (lanes 0-15: block b0, 16-31: block b1; lane = column c):
  // forward substitution T = (I + A_rr)^-1 column by column in fp32, then T - I to the ring.
  auto diag_solve = [&](int b0, int b1, __amdgpu_buffer_rsrc_t rr) {
    const int half = (lane >> 4) & 1, c = li;
    const float* A = Adiag[pw][half];
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (i == c) ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < 15; ++j) {
      const float xj = x[j];
#pragma unroll
      for (int i4 = (j + 1) / 4; i4 < 4; ++i4) {
        const float4 a = ld4f(&A[j * 16 + 4 * i4]);
        const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * i4 + e > j) x[4 * i4 + e] -= av[e] * xj;
      }
    }
    f16* Tw = Tt[pw][half];
    if (lane < 32) {
#pragma unroll
      for (int i = 0; i < 16; ++i) Tw[ta_off(i, c >> 2) + (c & 3)] = static_cast<f16>(x[i] - (i == c ? 1.f : 0.f));
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's transposed writes are done
    // lane (g, i) stores row i, piece g (8 bytes) of each block
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const f16x4 v = *reinterpret_cast<const f16x4*>(&Tt[pw][hb][ta_off(li, g4)]);
      st8(rr, (uint32_t)(kPkgTA + (ta_blk(hb ? b1 : b0, hb ? b1 : b0) * 256 + ta_off(li, g4)) * 2), v);
    }
  };

  if (w == 2 || w == 3) {
    // ================================================================== output waves (+ production)
    const int sw = w - 2;
    f32x4 Zp[4];  // Z^T of the previous chunk (value column 4g + r, token 16 tb + i)
    // production registers (tiles of this wave)
    bf16x8 fkA[KS], fkB[KS], fqA[KS], fqB[KS];  // pw 0: K/Q tiles 0 and 3; pw 1: tiles 1 and 2
    GateBits gbits{0, 0, 0, 0};
    const int tA = sw == 0 ? 0 : 1, tB = sw == 0 ? 3 : 2;
    for (int i = i_begin; i < i_end; ++i) {
      if (i >= 0 && i < nc) {
        // Z^T_i = S_i^T Q_i^T
        const f16* qb = Qc[i & 1];
        f16x8 sbv[KS], qf[KS][4];
#pragma unroll
        for (int s = 0; s < KS; ++s) sbv[s] = Sx[i & 1][sw][s * 64 + lane];
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) qf[s][tb] = ld8h(qb + (16 * tb + li) * KP + kq_col(s, li, g4));
        f32x4 Zt[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) Zt[tb] = f32x4{};
        // O of the previous chunk first (its operands are older)
        if (i >= 1) {
          const int c = i - 1;
          const f16* pp = Pc[c & 1];
          const f16x8 db0 = Dx[c & 1][sw][lane], db1 = Dx[c & 1][sw][64 + lane];
          f16x8 pf[6];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) pf[tb] = ld8h(pp + tp_off(16 * tb + li, 8 * g4));
          pf[4] = ld8h(pp + tp_off(32 + li, 32 + 8 * g4));
          pf[5] = ld8h(pp + tp_off(48 + li, 32 + 8 * g4));
          bf16* op = Ob[c & 1];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            f32x4 o = Zp[tb] * (p.scale * Gc[c % 3].egam[16 * tb + li]);
            o = mmah(db0, pf[tb], o);
            if (tb >= 2) o = mmah(db1, pf[tb + 2], o);
            *reinterpret_cast<bf16x4*>(op + vo_off(16 * tb + li, 16 * sw + 4 * g4)) = to_bf16x4(o[0], o[1], o[2], o[3]);
          }
        }
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) Zt[tb] = mmah(sbv[s], qf[s][tb], Zt[tb]);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) Zp[tb] = Zt[tb];
      } else if (i == nc && nc > 0) {
        const int c = nc - 1;
        const f16* pp = Pc[c & 1];
        const f16x8 db0 = Dx[c & 1][sw][lane], db1 = Dx[c & 1][sw][64 + lane];
        f16x8 pf[6];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) pf[tb] = ld8h(pp + tp_off(16 * tb + li, 8 * g4));
        pf[4] = ld8h(pp + tp_off(32 + li, 32 + 8 * g4));
        pf[5] = ld8h(pp + tp_off(48 + li, 32 + 8 * g4));
        bf16* op = Ob[c & 1];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          f32x4 o = Zp[tb] * (p.scale * Gc[c % 3].egam[16 * tb + li]);
          o = mmah(db0, pf[tb], o);
          if (tb >= 2) o = mmah(db1, pf[tb + 2], o);
          *reinterpret_cast<bf16x4*>(op + vo_off(16 * tb + li, 16 * sw + 4 * g4)) = to_bf16x4(o[0], o[1], o[2], o[3]);
        }
      }
      // ---- production of this slice's packages
      const int jA = i + kLead, jB = i + kLead - 1, jC = i + kLead - 2;
      if (jA < nc && jA % NVB == vb) {
        const auto rk = frag_rsrc(kg, jA), rq = frag_rsrc(qg, jA);
        load_tile(fkA, rk, tA);
        load_tile(fkB, rk, tB);
        load_tile(fqA, rq, tA);
        load_tile(fqB, rq, tB);
        fetch_gates(jA, gbits);
      } else if (jB >= 0 && jB < nc && jB % NVB == vb) {
        decide_wt();
        if (jB >= R) {
#pragma unroll
          for (int s = 0; s < NVB; ++s) wait_word(ack_off(jB % R, s), (unsigned)(jB - R + 1), dead);
        }
        if (l2) {
          norm_tile(fkA);
          norm_tile(fkB);
          norm_tile(fqA);
          norm_tile(fqB);
        }
        float gt[5];
        gate_terms(jB, gbits, gt);
        Gw[pw][0][lane] = gt[0];
        Gw[pw][1][lane] = gt[2];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        const auto rr = ring_rsrc(jB);
        // tiles: pw 0: (0,0) (3,0) (3,3); pw 1: (1,1) (2,1) (2,2)
        pg_tile(tA, tA, fkA, fqA, fkA, rr, Adiag[pw][0]);
        pg_tile(tB, tA, fkA, fqB, fkB, rr, nullptr);
        pg_tile(tB, tB, fkB, fqB, fkB, rr, Adiag[pw][1]);
      } else if (jC >= 0 && jC < nc && jC % NVB == vb) {
        const auto rr = ring_rsrc(jC);
        diag_solve(tA, tB, rr);
        raise_flag(jC);
      }
      __syncthreads();
    }
    return;
  }

  if (w >= 6) {
    // ================================================================== q/k staging (+ production)
    // Wave 6 stages K, wave 7 Q: the rows of chunk c + 1 loaded during step c - 1 ... converted
    // (and L2-normalised when asked) into slot (c + 1) % 2 during step c. Lane l handles the
    // 16-byte chunks l + 64 u of the tile: row (l + 64u) / 16, chunk (l + 64u) % 16.
    const bool is_k = w == 6;
    const bf16* src = is_k ? kg : qg;
    bf16x8 pr[16];
    auto fetch_rows = [&](int c) {
      const int64_t c0 = bos + (int64_t)c * kC;
      const auto rs = make_rsrc(src + (c0 * p.H + h) * KD, (uint32_t)chunk_len(c) * qk_row);
      const int tq = opaque_int(lane);
      const uint32_t base = (uint32_t)(tq / KCH) * qk_row + (uint32_t)(tq % KCH) * 16;
#pragma unroll
      for (int u = 0; u < 16; ++u) pr[u] = buf_load16(rs, base + (uint32_t)(u * (64 / KCH)) * qk_row);
    };
    auto stage_rows = [&](f16* dst) {  // row tq / 16 + 4u, chunk tq % 16 at its row's swizzle
      const int tq = opaque_int(lane);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int row = tq / KCH + u * (64 / KCH);
        *reinterpret_cast<f16x8*>(dst + row * KP + (((tq % KCH) ^ kq_sw(row)) << 3)) =
            bf16_to_f16x8(l2 ? l2norm_row_chunk<KCH>(pr[u]) : pr[u]);
      }
    };
    // production registers
    bf16x8 fk0[KS], fk1[KS], fk2[KS], fq0[KS], fq1[KS];
    GateBits gbits{0, 0, 0, 0};
    for (int i = i_begin; i < i_end; ++i) {
      if (i == -2 && nc > 0) fetch_rows(0);
      if (i >= -1 && i + 1 < nc) {  // chunk i + 1 into its slot, the loads of chunk i + 2
        stage_rows(is_k ? Kc[(i + 1) & 1] : Qc[(i + 1) & 1]);
        if (i + 2 < nc) fetch_rows(i + 2);
      }
      const int jA = i + kLead, jB = i + kLead - 1;
      if (jA < nc && jA % NVB == vb) {
        const auto rk = frag_rsrc(kg, jA), rq = frag_rsrc(qg, jA);
        if (pw == 2) {  // (1,0) (2,0): K tiles 0, 1, 2; Q tiles 1, 2
          load_tile(fk0, rk, 0);
          load_tile(fk1, rk, 1);
          load_tile(fk2, rk, 2);
          load_tile(fq0, rq, 1);
          load_tile(fq1, rq, 2);
        } else {  // (3,1) (3,2): K tiles 1, 2, 3; Q tile 3
          load_tile(fk0, rk, 1);
          load_tile(fk1, rk, 2);
          load_tile(fk2, rk, 3);
          load_tile(fq0, rq, 3);
        }
        fetch_gates(jA, gbits);
      } else if (jB >= 0 && jB < nc && jB % NVB == vb) {
        decide_wt();
        if (jB >= R) {
#pragma unroll
          for (int s = 0; s < NVB; ++s) wait_word(ack_off(jB % R, s), (unsigned)(jB - R + 1), dead);
        }
        if (l2) {
          norm_tile(fk0);
          norm_tile(fk1);
          norm_tile(fk2);
          norm_tile(fq0);
          if (pw == 2) norm_tile(fq1);
        }
        float gt[5];
        gate_terms(jB, gbits, gt);
        Gw[pw][0][lane] = gt[0];
        Gw[pw][1][lane] = gt[2];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        const auto rr = ring_rsrc(jB);
        if (pw == 2) {
          pg_tile(1, 0, fk0, fq0, fk1, rr, nullptr);
          pg_tile(2, 0, fk0, fq1, fk2, rr, nullptr);
          // the gate terms of the package (ChunkGates image: gam, egam, bet, begam, dlast)
#pragma unroll
          for (int x = 0; x < 5; ++x) st4(rr, (uint32_t)(kPkgG + (x * kC + lane) * 4), gt[x]);
        } else {
          pg_tile(3, 1, fk0, fq0, fk2, rr, nullptr);
          pg_tile(3, 2, fk1, fq0, fk2, rr, nullptr);
          // P above the diagonal is zero: tiles (rt, ct), ct > rt
#pragma unroll
          for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = rt + 1; ct < 4; ++ct)
              st8(rr, (uint32_t)(kPkgP + tp_off(16 * rt + li, tok_col(16 * ct + 4 * g4)) * 2), f16x4{});
        }
        raise_flag(jB);
      }
      __syncthreads();
    }
    return;
  }

  if (w == 4) {
    // ================================================================== package and V copies
    // During step i: the package of chunk i + 1 (T/A blocks, gate terms) once its four flags are
    // raised, P of chunk i, and the V slice of chunk i + 1; then the acknowledgement of chunk i.
    const int64_t vcol = vb * kVBc;
    for (int i = i_begin; i < i_end; ++i) {
      const int jn = i + 1;
      if (jn >= 0 && jn < nc) {
#pragma unroll
        for (int fw = 0; fw < 4; ++fw) wait_word(flag_off(jn % R, fw), (unsigned)(jn + 1), dead);
        const auto rr = make_rsrc(ring + (int64_t)(jn % R) * kSlotBytes, (uint32_t)kSlotBytes);
#pragma unroll
        for (int u = 0; u < 5; ++u)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(&TAc[jn & 1][0] + u * 512), 16,
                                                   (uint32_t)(kPkgTA + u * 1024 + lane * 16), 0, 0, kSC1);
#pragma unroll
        for (int u = 0; u < 5; ++u)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(reinterpret_cast<char*>(&Gc[jn % 3]) + u * 256), 4,
                                                   (uint32_t)(kPkgG + u * 256 + lane * 4), 0, 0, kSC1);
        // V slice rows 16 u + l / 4, 16-byte slot l % 4 of the LDS row receives source chunk slot ^ swizzle
        const int64_t c0 = bos + (int64_t)jn * kC;
        const auto rv = make_rsrc(vg + (c0 * p.HV + hv) * VD + vcol, (uint32_t)chunk_len(jn) * v_row);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int row = 16 * u + (lane >> 2), slot = lane & 3, ch = slot ^ ((row >> 2) & 3);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(&Vc[jn & 1][0] + u * 512), 16,
                                                   (uint32_t)(row * v_row + ch * 16), 0, 0, 0);
        }
      }
      if (i >= 0 && i < nc) {
        const auto rr = make_rsrc(ring + (int64_t)(i % R) * kSlotBytes, (uint32_t)kSlotBytes);
#pragma unroll
        for (int u = 0; u < 8; ++u)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(&Pc[i & 1][0] + u * 512), 16,
                                                   (uint32_t)(kPkgP + u * 1024 + lane * 16), 0, 0, kSC1);
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the copies have landed (the barrier publishes them)
      if (i >= 0 && i < nc && lane == 0)
        __builtin_amdgcn_raw_buffer_store_b32((unsigned)(i + 1), rsync, (int)ack_off(i % R, vb), 0, kSC1);
      __syncthreads();
    }
    return;
  }

  // ================================================================== wave 5: O stores
  // O of chunk c (written by the output waves during step c + 1) goes out during step c + 2:
  // lane l stores the 16-byte pieces l + 64 u (row (l + 64u) / 4, piece (l + 64 u) % 4), non-temporal.
  u16x2 om = {0, 0};
  for (int i = i_begin; i < i_end; ++i) {
    const int c = i - 2;
    if (c >= 0 && c < nc) {
      const int64_t c0 = bos + (int64_t)c * kC;
      const auto ro = make_rsrc(og + (c0 * p.HV + hv) * VD + vb * kVBc, (uint32_t)chunk_len(c) * v_row);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = lane + 64 * u, row = e >> 2, c8 = e & 3;
        const bf16x8 x = *reinterpret_cast<const bf16x8*>(&Ob[c & 1][vo_off(row, c8 * 8)]);
        const u32x4 wv = __builtin_bit_cast(u32x4, x);
#pragma unroll
        for (int q = 0; q < 4; ++q) om = __builtin_elementwise_max(om, __builtin_bit_cast(u16x2, wv[q] & 0x7fff7fffu));
        __builtin_amdgcn_raw_buffer_store_b128(wv, ro, (int)((uint32_t)row * v_row + c8 * 16), 0, 2);
      }
    }
    __syncthreads();
  }
  if (p.range_flag && (om[0] >= 0x7f80 || om[1] >= 0x7f80))
    __hip_atomic_store(p.range_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Zeroes the sync words of every chain (flags, acknowledgements, XCC ids): a fill kernel rather than
// a memset, so that a captured graph clears them on every replay.
__global__ __launch_bounds__(256) void gated_delta_chunk_sync_clear_kernel(unsigned* w, int64_t words) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < words; e += (int64_t)gridDim.x * 256) w[e] = 0u;
}

int coop_ring_slots(int64_t T) { return (int)std::min<int64_t>(kRing, std::max<int64_t>(1, (T + kC - 1) / kC)); }
int64_t coop_ring_bytes(int64_t chains, int64_t T) { return align256(chains * (int64_t)coop_ring_slots(T) * kSlotBytes); }
int64_t coop_sync_bytes(int64_t chains) { return align256((chains * (int64_t)(kHeadWords + kRing * kSyncWords) + 1) * 4); }

int launch_chunk_coop(const CoopArgs& a, hipStream_t s) {
  const int64_t chains = a.N * a.HV;
  const int64_t groups = (chains + 7) / 8;
  const int64_t blocks = groups * 8 * (128 / kVBc);
  if (blocks > 0x7fffffff) {
    gdn_internal_set_error("gdn_chunk_fwd: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  const int64_t words = chains * (kHeadWords + kRing * kSyncWords) + 1;  // + the error word
  const unsigned cgrid = (unsigned)std::min<int64_t>(256, (words + 255) / 256);
  hipLaunchKernelGGL(gated_delta_chunk_sync_clear_kernel, dim3(cgrid), dim3(256), 0, s, a.sync, words);
  unsigned* const err = a.err ? a.err : a.sync + (words - 1);  // the word after the chains' sync words
  CoopParams p{a.q, a.k, a.v, a.g, a.beta, a.h0, a.o, a.ht, a.cu, a.order, a.cu_i32, a.T, a.H, a.HV, a.N,
               a.dg, a.db, a.scale, a.flags, a.A_log, a.dt_bias, a.ring, coop_ring_slots(a.T), a.sync,
               a.range_flag, err};
  hipLaunchKernelGGL((gated_delta_chunk_coop_kernel<128, 128>), dim3((unsigned)blocks), dim3(kCoopNT), 0, s, p);
  return gdn_internal_check_launch("gated_delta_chunk_coop_kernel");
}

}  // namespace gdn
