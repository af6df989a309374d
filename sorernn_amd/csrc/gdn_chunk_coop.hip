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
// The roles run their own loops; after start-up there is no workgroup barrier, only LDS progress
// words (release / acquire at workgroup scope) that each role waits on, boundedly:
//   Waves 0, 1 (SIMDs 0, 1) -- the chain: Y = K S, X, the block substitution and the state update of
//     every chunk for 16 state columns each, S [K x 16] in fp32 MFMA accumulators for the whole
//     sequence. The operands of chunk i + 1 are read into registers during chunk i; Delta and the
//     fp16 S go to LDS for the output wave (ch_done).
//   Wave 2 -- the output of the 32 columns: O of chunk i - 1 (stored to HBM) and Z = S^T Q^T of i,
//     with Q of chunk i in registers, loaded from the ring one step ahead (out_done).
//   Wave 3 -- copies (buffer_load ... lds): K, the T/A blocks, the gate terms and V of chunk i + 2
//     and P of chunk i + 1 into LDS slots (rdy), the flag poll of package i + 3, the
//     acknowledgement of package i - 1.
//   Waves 4-7 -- package production, one package at a time, ahead of the chain by up to the ring.
// The package of a chunk -- its q/k rows L2-normalised (when asked) in fp16, P, the A blocks below
// the diagonal, T_rr - I and the gate terms -- is the same for the four slices. Slice (chunk % 4)
// builds it in a ring slot in L2 (the workspace): the four producing waves load and normalise one
// 16-row tile of q and k each (stored to the ring and, for k, to LDS), meet at an LDS arrival
// counter, form five 16 x 16 product tiles each (P row tile w - 4, A row tile 7 - w, one of them a
// diagonal A_rr), meet again, solve their diagonal block, and raise one flag each. A ring slot is
// reused kRing chunks later, once all four slices have acknowledged it.
//
// Performance (config 1 on one MI355X, measured): 151-156 us per call against 118-120 us for the
// two-kernel prefill (and 130 us against 96 us with a quarter of the chains), so the two-kernel
// prefill stays the default. The time per chunk is the chain's dependent latency plus the wait for
// the copy wave, whose 35 LDS copies per chunk take ~2.5k cycles to issue under load.
//
// Coherence. Within an XCD the L2 is the coherence point: the producer's plain stores reach it
// before its flag store (s_waitcnt vmcnt(0) between them), and consumers read flags and packages
// with device-scope (sc1) loads, which miss in the CU's L1. The four slices check at start-up,
// through write-through (sc1) stores, that they share an XCD; if not, the producers write with sc1
// stores (write-through to memory), which the consumers' sc1 loads see from any XCD. Every wait is
// bounded; a wait that runs out sets the error word and the range flag and the kernel completes.
//
// Precision: as the two-kernel prefill -- fp16 MFMA operands (S, X, Delta, T_rr - I, A, P, the
// bf16-rounded normalised q/k) with fp32 accumulation; the block substitution keeps b_r in the
// fp32 accumulator and rounds only the (T_rr - I) b_r operand (a CPU simulation at config-1
// statistics: final-state relative L2 2.19e-4, as with the full inverse).

#include <algorithm>
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

namespace {

constexpr int kCoopNT = 512;
constexpr int kVBc = 32;  // value columns per workgroup
constexpr int kRing = 8;  // packages in flight per chain
// package image in a ring slot (bytes): K rows, Q rows (the LDS images), P, the 10 T/A blocks, gates
constexpr int kPkgK = 0, kPkgQ = 16384, kPkgP = 32768, kPkgTA = 40960, kPkgG = 46080, kSlotBytes = 47360;
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

// Cache policy bits of the buffer instructions (gfx950): sc1 = device scope, nt = non-temporal.
constexpr int kSC1 = 16, kNT = 2;

// s_waitcnt immediates (gfx9 encoding, the other counters left at their maxima)
constexpr int kVmcnt0 = 0x0F70, kLgkmcnt0 = 0xC07F;
constexpr int kVmcnt35 = 0x8F73;  // vmcnt 35 = 0b10'0011: bits [3:0] = 3, bits [15:14] = 2

__device__ __forceinline__ bool all_reached(u32x4 v, unsigned want) {
  return (int)(v[0] - want) >= 0 && (int)(v[1] - want) >= 0 && (int)(v[2] - want) >= 0 && (int)(v[3] - want) >= 0;
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

  __shared__ __align__(16) f16 Kc[3][kC * KP];       // K of chunk c in slot c % 3 (fp16)
  __shared__ __align__(16) f16 TAc[3][10 * 256];     // T_rr - I and -A_rc of chunk c in slot c % 3
  __shared__ __align__(16) f16 Pc[3][kC * kC];       // scale * P of chunk c in slot c % 3 (tok_col, tp_off)
  __shared__ __align__(16) ChunkGates Gc[4];         // gate terms of chunk c in slot c % 4
  __shared__ __align__(16) bf16 Vc[3][kC * kVBc];    // V slice of chunk c in slot c % 3 (vo_off)
  __shared__ __align__(16) f16x8 Sx[2][2][KS * 64];  // S entering chunk c (fp16 pairs) of chain wave w, slot c % 2
  __shared__ __align__(16) f16x8 Dx[2][2][2 * 64];   // Delta of chunk c (fp16 pairs) of chain wave w, slot c % 2
  __shared__ __align__(16) f16 Xk[kC * KP];          // producers: normalised K rows of their package (fp16)
  __shared__ __align__(16) float Adiag[4][256];      // producers: A_rr (fp32, column-major) of wave 4 + x
  __shared__ __align__(16) float Gw[4][2][kC];       // producers: gam / beta of the package chunk
  // progress words (LDS): the roles run their own loops and wait only for these
  __shared__ int rdy;          // copy wave: chunks <= rdy copied to LDS (with P of chunk rdy - 1)
  __shared__ int ch_done[2];   // chain wave w: chunk ch_done[w] done (its Delta and the S after it published)
  __shared__ int out_done;     // output wave: step out_done done
  __shared__ int pbar;         // producing waves: arrivals at their group barrier

  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), g4 = lane >> 4, li = lane & 15;

  auto kq_sw = [](int r) { return (r & 7) << 1; };
  auto kq_col = [&](int s, int l_i, int l_g) { return (((4 * s + l_g) ^ kq_sw(l_i)) << 3); };
  auto tp_off = [](int r, int col) { return r * kC + ((((col >> 3) ^ (r & 7)) << 3) | (col & 7)); };
  auto vo_off = [](int r, int col) { return r * kVBc + ((((col >> 3) ^ ((r >> 2) & 3)) << 3) | (col & 7)); };
  // the K^T A operand of state tile a against token pair u (l_i, l_g: the lane's i and g)
  auto kt_pair = [&](const f16* tile, int u, int a, int l_i, int l_g) {
    const int m = l_i >> 2, q = l_i & 3;
    const int row = 32 * u + 4 * l_g + m;
    const f16* p0 = tile + row * KP + ((((4 * (a >> 1) + q) ^ kq_sw(4 * l_g + m)) << 3) + 4 * (a & 1));
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
  // the four flags (acks) of a slot are one 16-byte word group
  auto flags_off = [](int slot) { return (uint32_t)((kHeadWords + slot * kSyncWords) * 4); };
  auto acks_off = [](int slot) { return (uint32_t)((kHeadWords + slot * kSyncWords + 4) * 4); };

  // Bounded wait until the four sync words at `off` reach `want` (device-scope loads). `dead`
  // (uniform) short-cuts every later wait once one has run out.
  bool dead = false;
  auto wait4 = [&](uint32_t off, unsigned want) {
    if (dead) return;
    unsigned spins = 0;
    while (true) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsync, (int)off, 0, kSC1);
      if (__builtin_amdgcn_readfirstlane(all_reached(v, want) ? 1 : 0)) break;
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
  if (t == 0) __builtin_amdgcn_raw_buffer_store_b32(xcc_id() + 1, rsync, vb * 4, 0, kSC1);
  // V slots start as zeros; the copies write zeros for rows past a sequence's end (out-of-range
  // lanes of buffer_load ... lds), so every V row the chain reads is finite.
  for (int e = t; e < 3 * kC * kVBc / 8; e += kCoopNT) reinterpret_cast<bf16x8*>(&Vc[0][0])[e] = bf16x8{};
  if (t == 0) {
    rdy = -4;
    ch_done[0] = ch_done[1] = -2;
    out_done = -2;
    pbar = 0;
  }
  __syncthreads();  // the only workgroup barrier: from here on the roles synchronise through LDS words

  // Bounded wait until the LDS progress word *wp reaches `want` (acquire: the LDS data the word
  // publishes is read after it).
  auto wait_ge = [&](int* wp, int want) {
    unsigned spins = 0;
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(wp, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) < want &&
           !dead) {
      if (++spins >= kSpinMax) {
        dead = true;
        if (lane == 0) {
          __hip_atomic_store(p.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          if (p.range_flag) __hip_atomic_store(p.range_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
      }
      __builtin_amdgcn_s_sleep(1);
    }
  };
  auto wait_ready = [&](int c) { wait_ge(&rdy, c); };
  // publishes a progress word after the wave's earlier LDS writes (release)
  auto publish = [&](int* wp, int v) {
    if (lane == 0) __hip_atomic_store(wp, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  };

  if (w < 2) {
    // ================================================================== chain waves
    const int sw = w;
    // h0 / ht of the wave's 16 columns through buffer resources (none without h0 / ht: the loads
    // then read zeros); the per-lane offsets are formed where they are used, not kept in registers
    // across the chunk loop.
    const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD + vb * kVBc + 16 * sw;
    const auto rh0 = make_rsrc(p.h0 ? p.h0 + sbase : nullptr, p.h0 ? (uint32_t)(KD * VD * 4) : 0u);
    const auto rht = make_rsrc(p.ht ? p.ht + sbase : nullptr, p.ht ? (uint32_t)(KD * VD * 4) : 0u);
    auto s_off = [&](int a, int r) {  // byte offset of state element (key 32 s + 8 g + 4 hh + r, column li)
      return (uint32_t)(opaque_int((8 * g4 * VD + li) * 4) + ((32 * (a >> 1) + 4 * (a & 1) + r) * VD) * 4);
    };
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
    // Operands of a chunk read ahead, in the step before (its copies are published by rdy by then):
    // K as Y's A operands, the T/A blocks, V, beta and beta e^gam, gam of the last row.
    f16x8 kf[KS][4];
    f16x4 tb[10];
    bf16x4 vv[4];
    float4 bt[4], bg[4];
    float glast = 0.f;
    // the lane's i and g through an opaque value: the LDS offsets are formed where they are used,
    // not hoisted out of the loop (one register set per slot) and spilled
    auto read_k = [&](int c) {
      const int lq = opaque_int(lane), l_i = lq & 15, l_g = lq >> 4;
      const f16* kb = Kc[c % 3];
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int b = 0; b < 4; ++b) kf[s][b] = ld8h(kb + (16 * b + l_i) * KP + kq_col(s, l_i, l_g));
    };
    auto read_rest = [&](int c) {
      const int lq = opaque_int(lane), l_i = lq & 15, l_g = lq >> 4;
      const f16* ta = TAc[c % 3];
      const bf16* vp = Vc[c % 3];
      const ChunkGates& G = Gc[c % 4];
#pragma unroll
      for (int x = 0; x < 10; ++x) tb[x] = *reinterpret_cast<const f16x4*>(ta + x * 256 + ta_off(l_i, l_g));
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        vv[b] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4*)(vp + vo_off(16 * b + 4 * l_g + (l_i >> 2), 16 * sw + 4 * (l_i & 3))));
        bt[b] = ld4f(&G.bet[16 * b + 4 * l_g]);
        bg[b] = ld4f(&G.begam[16 * b + 4 * l_g]);
      }
      glast = G.gam[kC - 1];
    };
    // S from h0 (state tile a = 2s + hh: row 4g + r is key 32s + 8g + 4hh + r), published for the
    // output wave's chunk 0 (ch_done = -1), and the operands of chunk 0; then the chunks, each reading
    // the next chunk's operands (from a valid slot also after the last chunk).
#pragma unroll
    for (int a = 0; a < KT; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        S[a][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rh0, (int)s_off(a, r), 0, 0));
    make_sb();
    publish_s(0);
    publish(&ch_done[sw], -1);
    if (nc > 0) {
      wait_ready(0);
      read_rest(0);
      read_k(0);
    }
    for (int i = 0; i < nc; ++i) {
      {
        const int lq = opaque_int(lane), li = lq & 15, g4 = lq >> 4;
        const f16* kb = Kc[i % 3];
        const ChunkGates& G = Gc[i % 4];
        // ---- Y = K S (S in fp16 pairs), row block by row block
        f32x4 D[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          D[b] = f32x4{};
#pragma unroll
          for (int s = 0; s < KS; ++s) D[b] = mmah(kf[s][b], sb(s), D[b]);
        }
        __builtin_amdgcn_sched_barrier(0);
        // K^T and e^{gam_c - gam}, read while the Y products, X and the substitution run
        f16x8 ktf[KT][2];
#pragma unroll
        for (int a = 0; a < KT; ++a)
#pragma unroll
          for (int u = 0; u < 2; ++u) ktf[a][u] = kt_pair(kb, u, a, li, g4);
        float4 dl[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) dl[b] = ld4f(&G.dlast[16 * b + 4 * g4]);
        __builtin_amdgcn_sched_barrier(0);
        const float ec = __expf(glast);
#pragma unroll
        for (int a = 0; a < KT; ++a) S[a] *= ec;
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
        // the first token pair's update runs while blocks 2 and 3 finish
        f16x8 dt[2];
        {
          const f32x4 x0 = {dl[0].x * D[0][0], dl[0].y * D[0][1], dl[0].z * D[0][2], dl[0].w * D[0][3]};
          const f32x4 x1 = {dl[1].x * D[1][0], dl[1].y * D[1][1], dl[1].z * D[1][2], dl[1].w * D[1][3]};
          dt[0] = pack8h(x0, x1);
        }
        const f16x8 db0 = pack8h(D[0], D[1]);
        D[2] = mma16h(tb[ta_blk(2, 2)], pack4h(D[2]), D[2]);
#pragma unroll
        for (int a = 0; a < KT; ++a) S[a] = mmah(ktf[a][0], dt[0], S[a]);
        D[3] = mma16h(tb[ta_blk(3, 2)], pack4h(D[2]), D[3]);
        D[3] = mma16h(tb[ta_blk(3, 3)], pack4h(D[3]), D[3]);
        {
          const f32x4 x0 = {dl[2].x * D[2][0], dl[2].y * D[2][1], dl[2].z * D[2][2], dl[2].w * D[2][3]};
          const f32x4 x1 = {dl[3].x * D[3][0], dl[3].y * D[3][1], dl[3].z * D[3][2], dl[3].w * D[3][3]};
          dt[1] = pack8h(x0, x1);
        }
        const f16x8 db1 = pack8h(D[2], D[3]);
        // ---- S' = e^{gam_c} S + K^T Delta~ (second token pair)
#pragma unroll
        for (int a = 0; a < KT; ++a) S[a] = mmah(ktf[a][1], dt[1], S[a]);
        // ---- the next chunk's T/A, V and gates (their registers are free now); Delta and S' in fp16
        // for the output wave once it is done with the slots (its step i - 1); the next chunk's K
        // (in the registers K^T used)
        __builtin_amdgcn_sched_barrier(0);
        wait_ready(i + 1);
        read_rest(i + 1);
        __builtin_amdgcn_sched_barrier(0);
        wait_ge(&out_done, i - 1);
        Dx[i & 1][sw][lane] = db0;
        Dx[i & 1][sw][64 + lane] = db1;
        make_sb();
        publish_s((i + 1) & 1);
        publish(&ch_done[sw], i);
        __builtin_amdgcn_sched_barrier(0);
        read_k(i + 1);
      }
    }
    if (p.ht) {
      uint32_t smax = 0;
#pragma unroll
      for (int a = 0; a < KT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(S[a][r]), rht, (int)s_off(a, r), 0, 0);
          smax = max(smax, __float_as_uint(S[a][r]) & 0x7fffffffu);
        }
      if (p.range_flag && smax >= 0x7f800000u)
        __hip_atomic_store(p.range_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return;
  }

  if (w == 2) {
    // ================================================================== output wave
    // Step i: O_{i-1} = scale (e^gam Z_{i-1} + P Delta) stored to HBM, non-temporal, and
    // Z^T_i = S_i^T Q_i^T for both 16-column halves (lane (g, i): value columns 4g..4g+3 of the
    // half, token 16 tb + i), once the chain waves have published Delta_{i-1} and S_i. Q_i (the B
    // operands: lane (g, i) holds row 16 tb + i, keys 32 s + 8 g ..) comes from the ring during
    // step i - 1, after the copy wave has seen its package's flags.
    f32x4 Zp[2][4];
    f16x8 qf[KS][4];
    f16x8 pf[6];  // P of chunk i - 1 (the A operands of P Delta), read during step i - 1
    float eg[4];  // e^gam of chunk i - 1 at tokens 16 tb + i
    u16x2 om = {0, 0};
    auto read_p = [&](int cp) {
      const int lq = opaque_int(lane), l_i = lq & 15, l_g = lq >> 4;
      const f16* pp = Pc[cp % 3];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) pf[tb] = ld8h(pp + tp_off(16 * tb + l_i, 8 * l_g));
      pf[4] = ld8h(pp + tp_off(32 + l_i, 32 + 8 * l_g));
      pf[5] = ld8h(pp + tp_off(48 + l_i, 32 + 8 * l_g));
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) eg[tb] = Gc[cp % 4].egam[16 * tb + l_i];
    };
    auto load_q = [&](int c) {
      const auto rq = make_rsrc(ring + (int64_t)(c % R) * kSlotBytes + kPkgQ, (uint32_t)(kC * KP * 2));
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const int row = 16 * tb + li;
          const uint32_t off = (uint32_t)(row * KP + (((4 * s + g4) ^ kq_sw(row)) << 3)) * 2;
          qf[s][tb] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)off, 0, kSC1));
        }
    };
    if (nc > 0) {
      wait_ready(-1);  // the copy wave has seen the flags of package 0
      load_q(0);
    }
    for (int i = 0; i <= nc; ++i) {
      // the step's LDS reads in one batch: Delta of chunk i - 1 and S of chunk i (from the chain
      // waves' step i - 1); P and e^gam of chunk i - 1 were read during step i - 1
      const int c = i - 1;
      const bool o_step = i >= 1, z_step = i < nc;
      wait_ge(&ch_done[0], i - 1);
      wait_ge(&ch_done[1], i - 1);
      f16x8 dx[2][2], sx[KS][2];
      if (o_step) {
#pragma unroll
        for (int cs = 0; cs < 2; ++cs) {
          dx[cs][0] = Dx[c & 1][cs][lane];
          dx[cs][1] = Dx[c & 1][cs][64 + lane];
        }
      }
      if (z_step) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          sx[s][0] = Sx[i & 1][0][s * 64 + lane];
          sx[s][1] = Sx[i & 1][1][s * 64 + lane];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (o_step) {
        const int64_t c0 = bos + (int64_t)c * kC;
        const auto ro = make_rsrc(og + (c0 * p.HV + hv) * VD + vb * kVBc, (uint32_t)chunk_len(c) * v_row);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) eg[tb] *= p.scale;
#pragma unroll
        for (int cs = 0; cs < 2; ++cs) {
          const f16x8 db0 = dx[cs][0], db1 = dx[cs][1];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            f32x4 o = Zp[cs][tb] * eg[tb];
            o = mmah(db0, pf[tb], o);
            if (tb >= 2) o = mmah(db1, pf[tb + 2], o);
            const u32x2 ob = __builtin_bit_cast(u32x2, to_bf16x4(o[0], o[1], o[2], o[3]));
            om = __builtin_elementwise_max(om, __builtin_bit_cast(u16x2, ob[0] & 0x7fff7fffu));
            om = __builtin_elementwise_max(om, __builtin_bit_cast(u16x2, ob[1] & 0x7fff7fffu));
            __builtin_amdgcn_raw_buffer_store_b64(ob, ro, (int)((uint32_t)(16 * tb + li) * v_row + (16 * cs + 4 * g4) * 2),
                                                 0, kNT);
          }
        }
      }
      if (z_step) {
        f32x4 Zt[2][4];
#pragma unroll
        for (int cs = 0; cs < 2; ++cs)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) Zt[cs][tb] = f32x4{};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const f16x8 s0 = sx[s][0], s1 = sx[s][1];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            Zt[0][tb] = mmah(s0, qf[s][tb], Zt[0][tb]);
            Zt[1][tb] = mmah(s1, qf[s][tb], Zt[1][tb]);
          }
        }
#pragma unroll
        for (int cs = 0; cs < 2; ++cs)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) Zp[cs][tb] = Zt[cs][tb];
        wait_ready(i + 1);  // package i + 1's flags seen, P of chunk i landed
        if (i + 1 < nc) load_q(i + 1);
        read_p(i);
      }
      publish(&out_done, i);
    }
    if (p.range_flag && (om[0] >= 0x7f80 || om[1] >= 0x7f80))
      __hip_atomic_store(p.range_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return;
  }

  if (w == 3) {
    // ================================================================== copies
    // Step i, in this order: the waits for the slots it fills to be free; vmcnt(0) for the copies of
    // step i - 1 and rdy = i + 1 in LDS (the chain and output waves read chunk i + 1's operands
    // ahead once they see it; every package <= i + 2 has been seen complete); the flag poll of
    // package i + 3 (one 16-byte device-scope load); the copies of K, the T/A blocks and the gate
    // terms of chunk i + 2 and of P of chunk i + 1 from the ring, and of V of chunk i + 2 from HBM;
    // then vmcnt(35) -- loads complete in order, so this waits for the poll only and leaves the
    // step's 35 copies in flight across the barrier. The acknowledgement of package i - 1 (whose
    // copies and Q loads were consumed in step i - 1) ends the step. In the first and last steps of
    // a sequence (not every copy exists) the step waits for all its copies.
    const int64_t vcol = vb * kVBc;
    auto copy_pkg = [&](int jk) {  // K, T/A blocks and gates of chunk jk from the ring; V from HBM
      const char* slot = ring + (int64_t)(jk % R) * kSlotBytes;
      const auto rr = make_rsrc(slot, (uint32_t)kPkgG);
#pragma unroll
      for (int u = 0; u < 16; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(&Kc[jk % 3][0] + u * 512), 16,
                                                 (uint32_t)(kPkgK + u * 1024 + lane * 16), 0, 0, kSC1);
#pragma unroll
      for (int u = 0; u < 5; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(&TAc[jk % 3][0] + u * 512), 16,
                                                 (uint32_t)(kPkgTA + u * 1024 + lane * 16), 0, 0, kSC1);
      // the 1,280-byte gate image as 1,024 + 256 bytes: every lane of a copy to LDS writes its
      // bytes (zeros when its source is out of range), so no copy may reach past the slot
      const auto rg = make_rsrc(slot + kPkgG, (uint32_t)sizeof(ChunkGates));
      char* const gdst = reinterpret_cast<char*>(&Gc[jk % 4]);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void*)gdst, 16, (uint32_t)(lane * 16), 0, 0, kSC1);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void*)(gdst + 1024), 4, (uint32_t)(1024 + lane * 4), 0, 0, kSC1);
      // V slice rows 16 u + l / 4, 16-byte slot l % 4 of the LDS row receives source chunk slot ^ swizzle
      const int64_t c0 = bos + (int64_t)jk * kC;
      const auto rv = make_rsrc(vg + (c0 * p.HV + hv) * VD + vcol, (uint32_t)chunk_len(jk) * v_row);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int row = 16 * u + (lane >> 2), sl = lane & 3, ch = sl ^ ((row >> 2) & 3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(&Vc[jk % 3][0] + u * 512), 16,
                                                 (uint32_t)(row * v_row + ch * 16), 0, 0, 0);
      }
    };
    auto copy_p = [&](int jp) {  // P of chunk jp from the ring
      const auto rr = make_rsrc(ring + (int64_t)(jp % R) * kSlotBytes, (uint32_t)kPkgG);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(&Pc[jp % 3][0] + u * 512), 16,
                                                 (uint32_t)(kPkgP + u * 1024 + lane * 16), 0, 0, kSC1);
    };
    for (int i = -3; i <= nc; ++i) {
      // slots free: K, T/A and V of chunk i - 1 (chain step i - 1), gates and P of chunk i - 2
      // (output step i - 2, which also loaded Q of package i - 1 from the ring)
      wait_ge(&ch_done[0], i - 1);
      wait_ge(&ch_done[1], i - 1);
      wait_ge(&out_done, i - 2);
      // the previous step's copies (K, T/A, gates and V of chunk i + 1, P of chunk i) have landed
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      publish(&rdy, i + 1);
      const int jq = i + 3, jk = i + 2, jp = i + 1;
      if (jq < nc && jp >= 0) {
        // steady state, straight-line: poll, 35 copies, vmcnt(35)
        const u32x4 fl = __builtin_amdgcn_raw_buffer_load_b128(rsync, (int)flags_off(jq % R), 0, kSC1);
        copy_pkg(jk);
        copy_p(jp);
        __builtin_amdgcn_s_waitcnt(kVmcnt35);  // the poll and every earlier step's copies have landed
        if (!__builtin_amdgcn_readfirstlane(all_reached(fl, (unsigned)(jq + 1)) ? 1 : 0))
          wait4(flags_off(jq % R), (unsigned)(jq + 1));
      } else {
        // pipeline fill and drain: the same work, then vmcnt(0)
        if (jq >= 0 && jq < nc) wait4(flags_off(jq % R), (unsigned)(jq + 1));
        if (jk >= 0 && jk < nc) copy_pkg(jk);
        if (jp >= 0 && jp < nc) copy_p(jp);
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
      }
      const int ja = i - 1;
      wait_ge(&out_done, ja);  // Q of package ja is in the output wave's registers
      if (ja >= 0 && ja < nc && lane == 0)
        __builtin_amdgcn_raw_buffer_store_b32((unsigned)(ja + 1), rsync, (int)(acks_off(ja % R) + vb * 4), 0, kSC1);
    }
    return;
  }

  // ================================================================== package production (waves 4-7)
  // Wave 4 + x owns row tile x of the package chunk's q/k (normalising and storing it) and the
  // product tiles P (x, c <= x) (and the zero tiles (x, c > x) of P) and A (3 - x, c <= 3 - x):
  // five products per wave, one of them the diagonal A_rr whose inverse the wave solves.
  const int pw = w - 4, ra = 3 - pw;
  bool wt = false;  // write-through ring stores (set when the chain's slices are not on one XCD)
  bool wt_known = false;
  auto decide_wt = [&]() {
    if (wt_known) return;
    wait4(0u, 1u);
    const u32x4 ids = __builtin_amdgcn_raw_buffer_load_b128(rsync, 0, 0, kSC1);
    const bool same = ids[1] == ids[0] && ids[2] == ids[0] && ids[3] == ids[0];
    wt = !__builtin_amdgcn_readfirstlane(same ? 1 : 0);
    wt_known = true;
  };
  auto ring_rsrc = [&](int j) { return make_rsrc(ring + (int64_t)(j % R) * kSlotBytes, (uint32_t)kSlotBytes); };
  auto st16 = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, f16x8 v) {
    const u32x4 x = __builtin_bit_cast(u32x4, v);
    if (wt) __builtin_amdgcn_raw_buffer_store_b128(x, r, (int)off, 0, kSC1);
    else __builtin_amdgcn_raw_buffer_store_b128(x, r, (int)off, 0, 0);
  };
  auto st8 = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, f16x4 v) {
    const u32x2 x = __builtin_bit_cast(u32x2, v);
    if (wt) __builtin_amdgcn_raw_buffer_store_b64(x, r, (int)off, 0, kSC1);
    else __builtin_amdgcn_raw_buffer_store_b64(x, r, (int)off, 0, 0);
  };
  auto st4 = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    if (wt) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, kSC1);
    else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, 0);
  };

  // Fragment tile of a package chunk: lane (g, i) holds row 16 tt + i, keys 32 s + 8 g .. + 7 (bf16,
  // the q/k tensors as given); rows past the chunk read as zeros.
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
  // lanes i + 16, i + 32, i + 48 (summed with the cross-row lane swaps, no LDS); fp32 sums,
  // 1 / max(||x||, 1e-12) as rsq, rounded to bf16.
  auto norm_tile = [&](bf16x8 (&x)[KS]) {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)x[s][e] * (float)x[s][e];
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    ss = __uint_as_float(a[0]) + __uint_as_float(a[1]);  // lanes l and l ^ 16, in the same order on both
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    ss = __uint_as_float(b[0]) + __uint_as_float(b[1]);  // and l ^ 32
    const float inv = __builtin_amdgcn_rsqf(fmaxf(ss, 1e-24f));
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[s][e] = static_cast<bf16>((float)x[s][e] * inv);
  };
  // raw gate bits of chunk c for lane = token (a 32-bit and a 16-bit load per tensor through
  // resources sized to the dtype actually used, so that the one not used reads nothing)
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
  // One 16 x 16 product tile: rows j of K row tile c (A operand, kA) against the columns t of the
  // fragment tile b (B operand). The accumulator lane (g, i) holds t = 16 rt + i (rt: b's tile)
  // against j = 16 c + 4 g + r.
  auto product = [&](const f16x8 (&kA)[KS], const f16x8 (&b)[KS]) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mmah(kA[s], b[s], acc);
    return acc;
  };

  // Phase 2 of wave 4 + PW: the products P (PW, c), c <= PW, and A (3 - PW, c), c <= 3 - PW -- five
  // independent MFMA chains issued together -- then their epilogues and ring stores.
  f16x8 fq[KS];  // phase 1 -> 2: the normalised q rows of row tile pw, fp16
  auto phase2 = [&](int j, auto PWc) {
    constexpr int PW = decltype(PWc)::value, RA = 3 - PW;
    const auto rr = ring_rsrc(j);
    const int lq = opaque_int(lane), l_i = lq & 15, l_g = lq >> 4;
    const float* gam = Gw[PW][0];
    f16x8 kt[4][KS];  // K row tiles 0 .. max(PW, RA) (A operands; tile RA is also the B operand of the A products)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int s = 0; s < KS; ++s)
        if (c <= PW || c <= RA) kt[c][s] = ld8h(Xk + (16 * c + l_i) * KP + kq_col(s, l_i, l_g));
    float gjv[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 v = ld4f(&gam[16 * c + 4 * l_g]);
      gjv[c][0] = v.x;
      gjv[c][1] = v.y;
      gjv[c][2] = v.z;
      gjv[c][3] = v.w;
    }
    const int tp = 16 * PW + l_i, ta_t = 16 * RA + l_i;
    const float gtp = gam[tp], gta = gam[ta_t], bta = Gw[PW][1][ta_t];
    __builtin_amdgcn_sched_barrier(0);  // the loads above are one batch (one LDS round trip)
    f32x4 accP[PW + 1], accA[RA + 1];
#pragma unroll
    for (int c = 0; c <= PW; ++c) accP[c] = f32x4{};
#pragma unroll
    for (int c = 0; c <= RA; ++c) accA[c] = f32x4{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int c = 0; c <= PW; ++c) accP[c] = mmah(kt[c][s], fq[s], accP[c]);
#pragma unroll
      for (int c = 0; c <= RA; ++c) accA[c] = mmah(kt[c][s], kt[RA][s], accA[c]);
    }
    // P row tile PW: scale exp(gam_t - gam_j) q_t.k_j for j <= t; zero tiles above the diagonal.
    // exp of a masked-out pair is never formed (it may overflow).
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int j0c = 16 * c + 4 * l_g;
      const uint32_t off = (uint32_t)(kPkgP + tp_off(tp, tok_col(j0c)) * 2);
      if constexpr (true) {
        if (c <= PW) {
          float pv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const bool le = c < PW || j0c + r <= tp;
            const float e = __expf(le ? gtp - gjv[c][r] : 0.f);
            pv[r] = le ? p.scale * e * accP[c <= PW ? c : 0][r] : 0.f;
          }
          st8(rr, off, to_f16x4(pv[0], pv[1], pv[2], pv[3]));
        } else {
          st8(rr, off, f16x4{});
        }
      }
    }
    // A row tile RA: beta_t exp(gam_t - gam_j) k_t.k_j for j < t; -A below the diagonal block to
    // the ring, A_rr to LDS for the solve
#pragma unroll
    for (int c = 0; c <= RA; ++c) {
      const int j0c = 16 * c + 4 * l_g;
      float av[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool lt = c < RA || j0c + r < ta_t;
        const float e = __expf(lt ? gta - gjv[c][r] : 0.f);
        av[r] = lt ? bta * e * accA[c][r] : 0.f;
      }
      if (c < RA) {
        st8(rr, (uint32_t)(kPkgTA + (ta_blk(RA, c) * 256 + ta_off(l_i, l_g)) * 2),
            to_f16x4(-av[0], -av[1], -av[2], -av[3]));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) Adiag[PW][(4 * l_g + r) * 16 + l_i] = av[r];  // column j, row t
      }
    }
  };

  // The four producing waves meet at an LDS arrival counter (a barrier of their own) between
  // phases 1 and 2 (every wave's K rows are in Xk) and after phase 2 (every wave has read Xk).
  int pb_target = 0;
  auto pbarrier = [&]() {
    pb_target += 4;
    if (lane == 0) __hip_atomic_fetch_add(&pbar, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    wait_ge(&pbar, pb_target);
  };
  bf16x8 rk[KS], rq[KS];  // phase 0 -> 1: the raw q/k rows of row tile pw
  GateBits gbits{0u, 0u, 0u, 0u};
  for (int j = vb; j < nc; j += NVB) {
    // ---- phase 0: raw rows and gates
    load_tile(rk, frag_rsrc(kg, j), pw);
    load_tile(rq, frag_rsrc(qg, j), pw);
    fetch_gates(j, gbits);
    // ---- phase 1: normalise, round, store the rows; gate terms
    decide_wt();
    if (j >= R) wait4(acks_off(j % R), (unsigned)(j - R + 1));  // the slot's last package is consumed
    if (l2) {
      norm_tile(rk);
      norm_tile(rq);
    }
    {
      const auto rr = ring_rsrc(j);
      const int row = 16 * pw + li;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int off = row * KP + (((4 * s + g4) ^ kq_sw(row)) << 3);
        const f16x8 fk = bf16_to_f16x8(rk[s]);
        fq[s] = bf16_to_f16x8(rq[s]);
        st16(rr, (uint32_t)(kPkgK + off * 2), fk);
        st16(rr, (uint32_t)(kPkgQ + off * 2), fq[s]);
        *reinterpret_cast<f16x8*>(Xk + off) = fk;
      }
      float gt[5];
      gate_terms(j, gbits, gt);
      Gw[pw][0][lane] = gt[0];
      Gw[pw][1][lane] = gt[2];
      if (pw == 3) {
#pragma unroll
        for (int x = 0; x < 5; ++x) st4(rr, (uint32_t)(kPkgG + (x * kC + lane) * 4), gt[x]);
      }
    }
    pbarrier();
    // ---- phase 2: product tiles, the wave's tile list fixed at compile time
    switch (pw) {
      case 0: phase2(j, std::integral_constant<int, 0>{}); break;
      case 1: phase2(j, std::integral_constant<int, 1>{}); break;
      case 2: phase2(j, std::integral_constant<int, 2>{}); break;
      default: phase2(j, std::integral_constant<int, 3>{}); break;
    }
    pbarrier();
    // ---- phase 3: T_rr - I of block ra, row li per lane (the four lanes of a row compute it
    // alike), by right-looking back substitution: with y = row li of T, y[k] is final once the
    // columns above k are done, and then updates y[j] -= y[k] A[k][j] for every j < k (fp32).
    // The strictly lower A_rr is one batch of broadcast LDS reads. Then the wave's flag.
    {
      const float* A = Adiag[pw];
      float4 col[15][4];
#pragma unroll
      for (int jj = 0; jj < 15; ++jj)
#pragma unroll
        for (int r4 = (jj + 1) / 4; r4 < 4; ++r4) col[jj][r4] = ld4f(&A[jj * 16 + 4 * r4]);
      __builtin_amdgcn_sched_barrier(0);
      float y[16];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) y[jj] = (jj == li) ? 1.f : 0.f;
#pragma unroll
      for (int k = 15; k >= 1; --k) {
        const float yk = y[k];
#pragma unroll
        for (int jj = 0; jj < k; ++jj) {
          const float4 c4 = col[jj][k >> 2];
          y[jj] -= yk * ((k & 3) == 0 ? c4.x : (k & 3) == 1 ? c4.y : (k & 3) == 2 ? c4.z : c4.w);
        }
      }
      // lane (g, i) stores piece g of row i: T[i][4g .. 4g + 3] - I
      float pc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = g4 == 0 ? y[e] : g4 == 1 ? y[4 + e] : g4 == 2 ? y[8 + e] : y[12 + e];
        pc[e] = (4 * g4 + e == li) ? v - 1.f : v;
      }
      const auto rr = ring_rsrc(j);
      st8(rr, (uint32_t)(kPkgTA + (ta_blk(ra, ra) * 256 + ta_off(li, g4)) * 2), to_f16x4(pc[0], pc[1], pc[2], pc[3]));
      __builtin_amdgcn_s_waitcnt(kVmcnt0);  // every ring store of the package is in L2 (or memory)
      if (lane == 0) {
        const uint32_t off = flags_off(j % R) + pw * 4;
        if (wt) __builtin_amdgcn_raw_buffer_store_b32((unsigned)(j + 1), rsync, (int)off, 0, kSC1);
        else __builtin_amdgcn_raw_buffer_store_b32((unsigned)(j + 1), rsync, (int)off, 0, 0);
      }
    }
  }
}

// Zeroes the sync words of every chain (flags, acknowledgements, XCC ids): a fill kernel rather than
// a memset, so that a captured graph clears them on every replay.
__global__ __launch_bounds__(256) void gated_delta_chunk_sync_clear_kernel(unsigned* w, int64_t words) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < words; e += (int64_t)gridDim.x * 256) w[e] = 0u;
}

int launch_fill_zero(unsigned* w, int64_t words, hipStream_t s) {
  if (words <= 0) return GDN_OK;
  const unsigned grid = (unsigned)std::min<int64_t>(256, (words + 255) / 256);
  hipLaunchKernelGGL(gated_delta_chunk_sync_clear_kernel, dim3(grid), dim3(256), 0, s, w, words);
  return gdn_internal_check_launch("gated_delta_chunk_sync_clear_kernel");
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
