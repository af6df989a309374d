// The state kernel of the chunked gated delta rule forward (prefill) for gfx950: bf16 MFMA,
// 64-token chunks, the fp32 state held in MFMA accumulators across the whole sequence. T =
// (I + A)^-1 of every chunk comes from gated_delta_chunk_prep_kernel through the workspace.
//
// Per chunk of c <= 64 tokens with gam = in-chunk cumsum of g (sore/model/gdn_ref.py:17-21 in
// chunk form; the algebra is restated in oracle/gdn_oracle.py::_chunk_segment):
//   X     = diag(beta) V - diag(beta exp(gam)) K S              Delta = T X = X + (T - I) X
//   O     = scale (diag(exp(gam)) Q S + P Delta),  P_tj = exp(gam_t - gam_j) q_t.k_j  (j <= t)
//   S'    = exp(gam_c) S + K^T diag(exp(gam_c - gam)) Delta
//
// Work split: one workgroup of 8 waves per (sequence, value head, 32-column slice of V); the V/32
// slices of one (sequence, head) sit on one XCD, so the tiles they all read come from one L2.
//   State waves 0 and 1 each own 16 state columns, S_b [K x 16] in fp32 accumulators, and run the
//   whole recurrence of their columns: every operand that depends on the state (S itself, X,
//   Delta, Delta~) is an accumulator fragment used in place as the next MFMA's operand, so the
//   state never passes through LDS. Per chunk: Y = K S, X, Delta, O^T = scale(e^gam Z^T +
//   Delta^T P^T), the state update, then Z^T = S^T Q^T of the next chunk (60 MFMAs).
//   Helper waves 2-7 stage the chunk-wide operands one chunk ahead. Waves 2, 3, 6 and 7 (SIMDs 2
//   and 3, which hold no state wave) take the heavier work: q/k rows (L2-norm when asked, fp16
//   conversion) and the scaled P of the next chunk. Waves 4 and 5, which share SIMDs 0 and 1 with
//   the state waves, copy the T - I rows and the V slice, scan the gates (wave 4) and store O of
//   the previous chunk.
// One barrier per chunk separates the two sides. Each role runs its own chunk loop (the barrier counts
// match), so a role's loop-carried registers (the helpers' loads in flight for the next step, the
// state waves' accumulators) do not share one register allocation; the state loop is unrolled by six
// so that every LDS slot index is a compile-time constant.
//
// Fragment layouts (16x16x32 MFMA, lane (g, i), element r = 0..3 of an accumulator):
//   S tile a = 2s + h (s = 32-deep key step): row 4g + r is key 32s + 8g + 4h + r, so the pair
//     (S_2s, S_2s+1) in fp16 is the B operand of K S (keys 32s + 8g..+7) and the A operand of S^T Q^T;
//     the K^T operand of the update reads K columns in that order (ld8_tr_pair).
//   Y, X, Delta tile b: rows 16b + 4g + r (tokens), column i; pairs (2u, 2u+1) contract over the
//     tokens 32u + 4g + r and 32u + 16 + 4g + r, which is the column order of T - I and P (tok_col).
//   Z^T, O^T tile tb: row 4g + r is the wave's value column, column i the token 16tb + i.
//
// Precision: MFMA operands are fp16 (v_mfma_f32_16x16x32_f16) with fp32 accumulation. The bf16
// q/k (rounded to bf16 after the optional L2 norm, as the reference's bf16 pipeline holds them)
// convert to fp16 exactly, so P and the K products are exact products; S, X, Delta and T - I enter
// as fp16 (11-bit significand, 8x finer than bf16), which keeps the fp32 final state within about
// 3e-4 relative L2 over 64 chunks without splitting any operand. The operands' magnitudes must
// stay inside the fp16 range (65504): true of L2-normalised q/k, activation-scale v and the
// states they produce.
//
// LDS: K (3 slots), Q (2 slots), T - I, P, V and O (2 slots each), gate terms (3 slots).

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

struct ChunkParams {
  const void *q, *k, *v, *g, *beta;
  const float* h0;
  void* o;
  float* ht;
  const f16* tw;  // T - I rows from the prep kernel
  const void* cu;
  const int* order;  // with cu: sequences by length, longest first
  int cu_i32;
  int64_t T, H, HV, N;
  int dg, db;
  float scale;
  unsigned flags;
  const float *A_log, *dt_bias;
  bf16* hs;                  // SAVE only: the state entering each chunk, bf16 [chunks][HV][V][K] (transposed)
  const int* chunk_first;    // SAVE with cu: chunks before each sequence
  unsigned* range_flag;      // set to 1 when a stored output is inf or NaN (null: no check)
  // NORM only: the gated RMSNorm of O, applied by epilogue workgroups of the same launch
  // (gdn_chunk_fwd_gated_norm)
  const bf16* gate;          // [tokens][HV][V], the layer's output gate
  const float* nw;           // [V] norm weight
  float neps;
  int nsplit;                // 1: the reference's separate rmsnorm and silu(gate) roundings
  unsigned* prog;            // [chains][kProgStride]: chunks whose O each V / 32 slice has stored (zero at launch)
  int nq;                    // PERSIST only: groups of V / 32 workgroups
  int nprod;                 // NORM only: workgroups that run the chains' slices (the rest: epilogue)
};

// Cache policy bits of the buffer instructions (gfx950): sc1 = device scope, nt = non-temporal.
constexpr int kPolSC1 = 16, kPolNT = 2;
// s_waitcnt vmcnt(0) (gfx9 encoding, the other counters left at their maxima)
constexpr int kWaitVm0 = 0x0F70;
constexpr unsigned kEpiSpinMax = 1u << 21;  // NORM: polls of an epilogue workgroup before it gives up
// NORM: 32-bit words between the progress words of consecutive chains (each chain's NVB words in a
// 256-byte block of its own, so the epilogue workgroups' polls spread over memory channels)
constexpr int kProgStride = 64;
// NORM: words 16 .. 16 + kEpiPostMax - 1 of a chain's block hold the XCC ids (+ 1) its epilogue
// workgroups post at start-up
constexpr int kEpiPostBase = 16, kEpiPostMax = 48;
// The XCC (XCD) the wave runs on (hardware register XCC_ID).
__device__ __forceinline__ unsigned wave_xcc() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20); }
constexpr int kJobTab = 512;   // PERSIST: jobs per group held in LDS (the grid is used when no group needs more)

// Running maximum, per 16-bit half, of the magnitude bits of the bf16 values in x: a half at or
// above 0x7f80 (all-ones exponent) has seen an inf or a NaN.
__device__ __forceinline__ u16x2 bf16_mag_max(u16x2 m, const bf16x8& x) {
  const u32x4 w = __builtin_bit_cast(u32x4, x);
#pragma unroll
  for (int i = 0; i < 4; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7fff7fffu));
  return m;
}

// Records a non-finite output: a system-scope vector store, so that a host word registered with
// gdn_set_range_flag sees it without a device-wide synchronisation.
__device__ __forceinline__ void flag_nonfinite(unsigned* flag, bool bad) {
  if (bad) __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr int kVB = 32;       // value columns per workgroup (two state waves of 16)
constexpr int kNT = 512;      // threads per workgroup (8 waves)

// SAVE (training forward): the state waves also store the state entering every chunk, rounded to
// bf16 and transposed ([V][K]: a lane's four consecutive keys are one 8-byte store), the input of
// the backward's per-chunk gradient kernel, which uses it only as a bf16 MFMA operand.
// workgroup -> (chain rank k, slice vb) -> (sequence n, value head hv). Workgroups are dispatched
// in blockIdx order and blockIdx b lands on XCD b % 8: XCD x takes chain ranks x, x + 8, ..., all
// NVB slices of a chain on one XCD (its q/k tiles are then read from one L2). Chain ranks follow
// the longest-first sequence order with cu_seqlens, so a grid larger than the machine starts the
// longest recurrences first.
struct SliceLoc {
  int64_t k;            // chain rank
  int64_t n, bos, eos;  // sequence and its token range
  int hv, h, vb;        // value head, its q/k head, V slice
};
template <int NVB>
__device__ __forceinline__ SliceLoc locate_slice(const ChunkParams& p) {
  const int64_t chains = p.N * p.HV;
  int64_t k_rank;
  SliceLoc l;
  if (chains % 8 == 0) {
    const int64_t x = blockIdx.x % 8, j = blockIdx.x / 8;
    k_rank = 8 * (j / NVB) + x;
    l.vb = (int)(j % NVB);
  } else {
    k_rank = blockIdx.x / NVB;
    l.vb = (int)(blockIdx.x % NVB);
  }
  l.k = k_rank;
  l.hv = (int)(k_rank % p.HV);
  l.n = p.order ? (int64_t)p.order[k_rank / p.HV] : k_rank / p.HV;
  l.h = l.hv / (int)(p.HV / p.H);
  if (p.cu) {
    l.bos = load_index(p.cu, p.cu_i32, l.n);
    l.eos = load_index(p.cu, p.cu_i32, l.n + 1);
  } else {
    l.bos = l.n * p.T;
    l.eos = l.bos + p.T;
  }
  return l;
}

// The kernel's parameters read again from the kernarg segment (the chunk kernel's only argument sits
// at offset 0), through an address the optimiser cannot see through: code that runs after the main
// loops (the recovery) then loads them where it runs, instead of keeping them in scalar registers
// through the loops.
__device__ __forceinline__ ChunkParams reload_params() {
  static_assert(sizeof(ChunkParams) % 8 == 0, "read as 8-byte words");
  constexpr int kWords = sizeof(ChunkParams) / 8;
  typedef const __attribute__((address_space(4))) uint64_t* kwords;
  uint64_t a = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
  asm volatile("" : "+s"(a));
  struct Words {
    uint64_t w[kWords];
  } r;
#pragma unroll
  for (int i = 0; i < kWords; ++i) r.w[i] = reinterpret_cast<kwords>(a)[i];
  return __builtin_bit_cast(ChunkParams, r);
}

// The fp32 recurrence of one 32-column slice of a (sequence, value head), per token (the algebra of
// gated_delta_recurrent_kernel, sore/model/gdn_ref.py:17-21):
//   a = exp(g), delta = beta (v - a S^T k^), S' = a S + k^ delta^T, o = scale S'^T q^
// with k^, q^ the fp32 L2-normalised k and q when asked. Wave w owns the columns 4w .. 4w + 3 of the
// slice: lane (g, i) holds rows i * KD/16 .. +KD/16 of column 4w + g, and the column's dot products
// are sums over its 16 lanes (DPP). Each chunk's q/k rows, V slice and gate values are staged in
// LDS (the chunk kernel's tiles, no longer in use) by all 512 threads first.
template <int KD, int VD, bool SAVE>
__device__ __forceinline__ void recover_slice(const ChunkParams& p, int64_t n, int hv, int h, int vb, int64_t bos,
                                           int64_t eos, int64_t cg_first, bf16* kl, bf16* ql, bf16* vl,
                                           ChunkGates* gl, int c_out_from = 0) {
  constexpr int KPL = KD / 16;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, g4 = lane >> 4, li = lane & 15;
  const int col = vb * kVB + 4 * w + g4;  // value column within the head
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const int64_t sb0 = (n * p.HV + hv) * (int64_t)KD * VD;
  float s[KPL];
#pragma unroll
  for (int e = 0; e < KPL; ++e) s[e] = p.h0 ? p.h0[sb0 + (int64_t)(li * KPL + e) * VD + col] : 0.f;
  const bf16* qg = static_cast<const bf16*>(p.q);
  const bf16* kg = static_cast<const bf16*>(p.k);
  const bf16* vg = static_cast<const bf16*>(p.v);
  bf16* og = static_cast<bf16*>(p.o);
  u16x2 om = {0, 0};
  const int nc = (int)((eos - bos + kC - 1) / kC);
  for (int c = 0; c < nc; ++c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    const int len = (int)((eos - c0) < kC ? (eos - c0) : kC);
    if constexpr (SAVE) {
      // the state entering chunk c, bf16, [V][K] (as the chunk kernel saves it)
      bf16* hs = p.hs + ((cg_first + c) * p.HV + hv) * (int64_t)(KD * VD) + (int64_t)col * KD + li * KPL;
#pragma unroll
      for (int e = 0; e < KPL; ++e) hs[e] = static_cast<bf16>(s[e]);
    }
    __syncthreads();  // the previous chunk's tiles are consumed
    for (int e = t; e < kC * KD; e += kNT) {
      const int r = e / KD, x = e % KD;
      const bool in = r < len;
      kl[e] = in ? kg[((c0 + r) * p.H + h) * KD + x] : bf16{};
      ql[e] = in ? qg[((c0 + r) * p.H + h) * KD + x] : bf16{};
    }
    for (int e = t; e < kC * kVB; e += kNT) {
      const int r = e / kVB, x = e % kVB;
      vl[e] = r < len ? vg[((c0 + r) * p.HV + hv) * VD + vb * kVB + x] : bf16{};
    }
    if (t < kC) {
      float a = 1.f, b = 0.f;
      if (t < len) {
        const int64_t idx = (c0 + t) * p.HV + hv;
        float gvv = load_as_f32(p.g, p.dg, idx);
        if (p.flags & GDN_FLAG_GATE_IN_KERNEL) gvv = -expf(p.A_log[hv]) * softplus_f32(gvv + p.dt_bias[hv]);
        a = expf(gvv);
        const float bv = load_as_f32(p.beta, p.db, idx);
        b = (p.flags & GDN_FLAG_BETA_SIGMOID) ? sigmoid_f32(bv) : bv;
      }
      gl->gam[t] = a;
      gl->bet[t] = b;
    }
    __syncthreads();
    for (int r = 0; r < len; ++r) {
      float kr[KPL], qr[KPL];
#pragma unroll
      for (int e = 0; e < KPL; ++e) {
        kr[e] = (float)kl[r * KD + li * KPL + e];
        qr[e] = (float)ql[r * KD + li * KPL + e];
      }
      const float a = gl->gam[r], b = gl->bet[r], vv = (float)vl[r * kVB + 4 * w + g4];
      float pk = 0.f, pq = 0.f, kq = 0.f, kk = 0.f, qq = 0.f;
#pragma unroll
      for (int e = 0; e < KPL; ++e) {
        pk += s[e] * kr[e];
        pq += s[e] * qr[e];
        kq += kr[e] * qr[e];
        kk += kr[e] * kr[e];
        qq += qr[e] * qr[e];
      }
      pk = group_sum<16>(pk);
      pq = group_sum<16>(pq);
      kq = group_sum<16>(kq);
      kk = group_sum<16>(kk);
      qq = group_sum<16>(qq);
      // F.normalize semantics: x / max(||x||, 1e-12)
      const float ik = l2 ? 1.f / fmaxf(sqrtf(kk), 1e-12f) : 1.f;
      const float iq = l2 ? 1.f / fmaxf(sqrtf(qq), 1e-12f) : 1.f;
      const float d = b * (vv - a * pk * ik);
      const float o = p.scale * (a * pq * iq + d * kq * ik * iq);
#pragma unroll
      for (int e = 0; e < KPL; ++e) s[e] = a * s[e] + kr[e] * ik * d;
      if (li == 0 && c >= c_out_from) {
        const bf16 ob = static_cast<bf16>(o);
        og[(c0 + r) * p.HV * VD + (int64_t)hv * VD + col] = ob;
        om = __builtin_elementwise_max(om, u16x2{(unsigned short)(__builtin_bit_cast(unsigned short, ob) & 0x7fff), 0});
      }
    }
  }
  uint32_t smax = 0;
  if (p.ht) {
#pragma unroll
    for (int e = 0; e < KPL; ++e) {
      p.ht[sb0 + (int64_t)(li * KPL + e) * VD + col] = s[e];
      smax = max(smax, __float_as_uint(s[e]) & 0x7fffffffu);
    }
  }
  if (p.range_flag) flag_nonfinite(p.range_flag, smax >= 0x7f800000u || om[0] >= 0x7f80);
}

constexpr int kLptMax = 128;  // PERSIST: sequences scheduled by rows (LPT); more go in snake order
struct SchedScratch {
  int nch[kLptMax], bos[kLptMax], eos[kLptMax], seq[kLptMax];  // the sequence of rank d (longest first)
  int ne;                                                        // non-empty sequences
};

// PERSIST: the job list of group gq, into jtab, by every thread of the workgroup (all groups compute
// the same schedule from the index kernel's longest-first order, each keeping its own list):
//   rows (HV divides the group count and at most kLptMax sequences): every value head of a
//   sequence goes to one row of HV groups, head h to the row's h-th group, so the groups of a row
//   carry equal loads, and wave 0 deals the sequences, longest first, each to the least-loaded row
//   (LPT; over the reference's document lengths the busiest group gets 135 chunks against a mean
//   of 134.5, against 157 in snake order);
//   otherwise the chains of the non-empty sequences in snake order (rank r: sequence order[r / HV],
//   head r % HV; job k of group q is rank k nq + q for even k, k nq + nq - 1 - q for odd k).
// gjob = (jobs, chunks in all of them). Empty sequences (last in the order) are in no list.
__device__ __forceinline__ void schedule_group(const ChunkParams& p, int gq, int4* jtab, int* gjob, SchedScratch& sc) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int N = (int)p.N, HV = (int)p.HV, nq = p.nq;
  const bool by_rows = nq % HV == 0 && N <= kLptMax;
  if (t == 0) {
    sc.ne = 0;
    gjob[0] = gjob[1] = 0;
  }
  __syncthreads();
  for (int d = t; d < N; d += kNT) {
    const int sq = p.order[d];
    const int64_t b = load_index(p.cu, p.cu_i32, sq), e = load_index(p.cu, p.cu_i32, sq + 1);
    if (by_rows) {
      sc.seq[d] = sq;
      sc.bos[d] = (int)b;
      sc.eos[d] = (int)e;
      sc.nch[d] = (int)((e - b + kC - 1) / kC);
    }
    if (e > b) atomicAdd(&sc.ne, 1);
  }
  __syncthreads();
  const int ne = sc.ne;
  if (by_rows) {
    if (w == 0) {
      // lane r < R holds row r's load; the least-loaded row is the minimum of (load << 6 | lane)
      // (loads stay below 2^25 chunks, so the keys stay positive)
      const int R = nq / HV, my_row = gq / HV, h = gq % HV;
      int load = lane < R ? 0 : 0x1ffffff, nj = 0, steps = 0, blk = 0;
      if (R <= 8) {
        // up to 8 rows: their loads in scalar registers (uniform code, no cross-lane steps)
        int ld[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int d = 0; d < ne; ++d) {
          if ((d & 63) == 0) blk = d + lane < ne ? sc.nch[d + lane] : 0;
          const int ncd = __builtin_amdgcn_readlane(blk, d & 63);
          int row = 0, best = ld[0];
#pragma unroll
          for (int r = 1; r < 8; ++r)
            if (r < R && ld[r] < best) {
              best = ld[r];
              row = r;
            }
#pragma unroll
          for (int r = 0; r < 8; ++r) ld[r] += r == row ? ncd : 0;
          if (row == my_row) {
            if (lane == 0) jtab[nj] = make_int4(sc.bos[d], sc.eos[d], sc.seq[d], h);
            ++nj;
            steps += ncd;
          }
        }
        if (lane == 0) {
          gjob[0] = nj;
          gjob[1] = steps;
        }
      }
      for (int d = 0; R > 8 && d < ne; ++d) {
        if ((d & 63) == 0) blk = d + lane < ne ? sc.nch[d + lane] : 0;
        const int ncd = __builtin_amdgcn_readlane(blk, d & 63);
        int key = (load << 6) | lane;
        key = min(key, __builtin_amdgcn_mov_dpp(key, 0xb1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
        key = min(key, __builtin_amdgcn_mov_dpp(key, 0x4e, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
        key = min(key, __builtin_amdgcn_mov_dpp(key, 0x141, 0xf, 0xf, false));  // row_half_mirror
        key = min(key, __builtin_amdgcn_mov_dpp(key, 0x140, 0xf, 0xf, false));  // row_mirror
        const int m = min(min(__builtin_amdgcn_readlane(key, 0), __builtin_amdgcn_readlane(key, 16)),
                          min(__builtin_amdgcn_readlane(key, 32), __builtin_amdgcn_readlane(key, 48)));
        const int row = m & 63;
        if (row == my_row) {
          if (lane == 0) jtab[nj] = make_int4(sc.bos[d], sc.eos[d], sc.seq[d], h);
          ++nj;
          steps += ncd;
        }
        if (lane == row) load += ncd;
      }
      if (R > 8 && lane == 0) {
        gjob[0] = nj;
        gjob[1] = steps;
      }
    }
  } else {
    const int64_t chains = (int64_t)ne * HV;
    for (int k = t; k < kJobTab; k += kNT) {
      const int64_t r = (int64_t)k * nq + ((k & 1) ? nq - 1 - gq : gq);
      if (r >= chains) break;
      const int sq = p.order[r / HV];
      const int64_t b = load_index(p.cu, p.cu_i32, sq), e = load_index(p.cu, p.cu_i32, sq + 1);
      jtab[k] = make_int4((int)b, (int)e, sq, (int)(r % HV));
      atomicAdd(&gjob[1], (int)((e - b + kC - 1) / kC));
      atomicMax(&gjob[0], k + 1);
    }
  }
  __syncthreads();
}

// PERSIST (inference with cu_seqlens and many chains, no initial or final state: the reference
// model's call): one workgroup per CU; the V / 32 workgroups of a group (on one XCD) walk the group's
// job list, a sequence of (sequence, value head) chains of their V-slice, back to back: every role
// treats the jobs' chunks as one stream of steps, so a short sequence does not pay a workgroup's
// pipeline fill and drain. At the last step of a job the state waves zero the state. (Storing and
// loading states there, in each of the six unrolled steps, made the kernel's code larger than the
// instruction cache two CUs share; calls with states keep one workgroup per slice.)
// NORM: epilogue workgroup j of nw (placed after the chains' slices in the grid, on CUs the slices
// leave free) applies the gated RMSNorm to O tiles of 64 tokens x V columns, in place:
// y = o rstd w silu(gate), rstd = 1 / sqrt(mean(o^2) + eps) over the head's V values of the rounded
// o, fp32 math and one rounding (FLA rms_norm_gated(o, gate, w, None, "swish", eps)); with nsplit
// the norm and silu(gate) are each rounded to bf16 before their product, as o_norm(o) * F.silu(gate)
// does. The arithmetic is the norm kernel's (gated_delta_norm_v8_kernel: a lane's 8 values, then
// the row's lane group), so the outputs equal those of the chunk kernel followed by that kernel.
// The host gives at least two epilogue workgroups per chain: R = nw / chains of them share a chain,
// workgroup j taking the chunks j / chains, + R, + 2R, ... of the chain with dispatch rank j % chains
// (in the order the slices store them). With the chain count a multiple of 8 the workgroup then runs
// on the XCD of its chain's slices (blockIdx b on XCD b % 8); it posts its XCC id at start-up, and a
// slice whose epilogue workgroups all share its XCD stores O to L2 only (the workgroups' device-scope
// loads are served there), otherwise written through to memory. Wave 0 polls the chain's V / 32 progress words (device-scope loads, a sleep
// of ~2k cycles between polls) until they pass the chunk, and a barrier releases the workgroup's
// eight waves, each of which handles its own rows of the tile. The polls are what the slices feel
// of the epilogue: at config 4, one polling wave per workgroup and a few polls per chunk keep the
// call at 206 us against 186 us for the chunk kernel alone (559 us with every wave polling every
// ~100 cycles, the polls queueing on the memory channel that held the words). The gate loads and
// y stores are non-temporal, leaving L2 to the slices' tiles. A wait that runs out sets the range
// flag, and the workgroup stops waiting.
template <int VD>
__device__ void norm_epilogue(const ChunkParams& p, int j, int nw) {
  constexpr int NVB = VD / kVB, LPR = VD / 8, RPW = kWave / LPR, NWV = kNT / kWave, U = kC / (RPW * NWV);
  static_assert(U * RPW * NWV == kC, "a tile's rows divide among the waves");
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, sub = lane / LPR, li = lane % LPR;
  const int64_t chains = p.N * p.HV, R = nw / chains;
  if (R < 1 || j >= R * chains) return;
  const int64_t kr = j % chains, n = p.order ? (int64_t)p.order[kr / p.HV] : kr / p.HV, hv = kr % p.HV;
  const int64_t ch = n * p.HV + hv;
  if (threadIdx.x == 0 && j / chains < kEpiPostMax) {
    const auto rb = make_rsrc(p.prog + ch * kProgStride, kProgStride * 4);
    __builtin_amdgcn_raw_buffer_store_b32(wave_xcc() + 1, rb, (int)((kEpiPostBase + j / chains) * 4), 0, kPolSC1);
  }
  int64_t bos, eos;
  if (p.cu) {
    bos = load_index(p.cu, p.cu_i32, n);
    eos = load_index(p.cu, p.cu_i32, n + 1);
  } else {
    bos = n * p.T;
    eos = bos + p.T;
  }
  float wv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) wv[e] = p.nw[li * 8 + e];
  const uint32_t vrow = (uint32_t)(p.HV * VD * 2);
  bf16* const og = static_cast<bf16*>(p.o);
  // lanes 0..NVB-1 of wave 0 read the slices' words; the other lanes' offsets are past the resource
  const auto rp = make_rsrc(p.prog + ch * kProgStride, NVB * 4);
  bool dead = false;  // wave 0: a wait ran out
  for (int64_t c = j / chains; bos + c * kC < eos; c += R) {
    const int64_t c0 = bos + c * kC;
    const uint32_t len = (uint32_t)min<int64_t>(kC, eos - c0);
    if (w == 0) {
      unsigned spins = 0;
      while (!dead) {
        const unsigned got = __builtin_amdgcn_raw_buffer_load_b32(rp, lane * 4, 0, kPolSC1);
        if (__builtin_amdgcn_ballot_w64(lane < NVB && got < (unsigned)(c + 1)) == 0) break;
        if (++spins >= kEpiSpinMax) {
          dead = true;
          if (lane == 0 && p.range_flag) flag_nonfinite(p.range_flag, true);
          break;
        }
        __builtin_amdgcn_s_sleep(32);
      }
    }
    __syncthreads();  // the tile is stored (or wave 0 gave up)
    // O rows through device-scope loads (written through by the slices on any XCD); rows past
    // len read as zeros and their stores are dropped (buffer range)
    const auto ro = make_rsrc(og + (c0 * p.HV + hv) * VD, len * vrow);
    const auto rg = make_rsrc(p.gate + (c0 * p.HV + hv) * VD, len * vrow);
    u32x4 xo[U], xg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = (u * NWV + w) * RPW + sub;
      xo[u] = __builtin_amdgcn_raw_buffer_load_b128(ro, (int)((uint32_t)row * vrow + li * 16), 0, kPolSC1);
      xg[u] = __builtin_amdgcn_raw_buffer_load_b128(rg, (int)((uint32_t)row * vrow + li * 16), 0, kPolNT);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = (u * NWV + w) * RPW + sub;
      const bf16x8 xv = __builtin_bit_cast(bf16x8, xo[u]), gvv = __builtin_bit_cast(bf16x8, xg[u]);
      float xf[8], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xf[e] = (float)xv[e];
        ss += xf[e] * xf[e];
      }
      ss = group_sum<LPR>(ss);
      const float scale = __builtin_amdgcn_rsqf(ss / (float)VD + p.neps);
      bf16x8 y;
      if (p.nsplit) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float y1 = (float)static_cast<bf16>(xf[e] * scale * wv[e]);
          y[e] = static_cast<bf16>(y1 * (float)static_cast<bf16>(silu_fast((float)gvv[e])));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = static_cast<bf16>(xf[e] * scale * wv[e] * silu_fast((float)gvv[e]));
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, y), ro, (int)((uint32_t)row * vrow + li * 16), 0,
                                             kPolNT);
    }
  }
}

template <int KD, int VD, bool SAVE, bool NORM = false, bool PERSIST = false>
__global__ __launch_bounds__(kNT, 1) void gated_delta_chunk_kernel(ChunkParams p) {
  static_assert(!(SAVE && NORM), "the fused norm is an inference epilogue");
  static_assert(!(PERSIST && (SAVE || NORM)), "the persistent grid runs plain inference calls");
  constexpr int NVB = VD / kVB;
  // q/k tiles in LDS: at KD = 128 rows are unpadded (256 B) and the 16-byte chunk c of row r sits
  // at chunk c ^ kq_sw(r) = c ^ ((r & 7) << 1). Measured with SQ_LDS_BANK_CONFLICT on gfx950, the
  // row-fragment reads (16 rows, one chunk) and the staging writes are then conflict-free and the
  // transposed K^T reads take 2 extra cycles per instruction; at KD = 64 rows are padded by 16 bytes.
  constexpr bool SWZ = KD == 128;
  constexpr int KP = SWZ ? KD : KD + 8;       // element pitch of the q/k tiles
  constexpr int KS = KD / 32;                 // MFMA k-steps over the key dim
  constexpr int KT = KD / 16;                 // 16-row state tiles
  constexpr int KCH = KD / 8;                 // 16-byte chunks per q/k row
  constexpr int QKPT = kC * KCH / 256;        // 16-byte chunks per thread of a q or k tile (waves 2, 3, 6, 7)

  __shared__ __align__(16) f16 Kc[3][kC * KP];   // K of chunk c in slot c % 3 (fp16)
  __shared__ __align__(16) f16 Qc[2][kC * KP];   // Q of chunk c in slot c % 2 (fp16)
  __shared__ __align__(16) f16 Tb[2][kC * kC];    // T - I of chunk c in slot c % 2 (tok_col columns, tp_off)
  __shared__ __align__(16) f16 Pb[2][kC * kC];    // scale * P of chunk c in slot c % 2 (tok_col columns, tp_off)
  __shared__ __align__(16) bf16 Vc[2][kC * kVB];  // V slice of chunk c in slot c % 2 (vo_off)
  // O of chunk c, stored to HBM during chunk c + 1 (slot c % 2)
  __shared__ __align__(16) bf16 Ob[2][kC * kVB];
  __shared__ __align__(16) ChunkGates gv[3];      // gate terms of chunk c in slot c % 3
  __shared__ int bad;                              // an O or final-state element of this slice is inf / NaN
  __shared__ int first_bad;                        // NORM: the first chunk whose stored O holds an inf or NaN
  __shared__ int4 jtab[PERSIST ? kJobTab : 1];     // PERSIST: the group's job list (bos, eos, sequence, head)
  __shared__ SchedScratch sched;                   // PERSIST: the scheduler's per-sequence arrays

  // w is read back as a scalar: the compiler then treats the role branches as wave-uniform
  const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6), g4 = lane >> 4, li = lane & 15;
  if constexpr (NORM) {
    if ((int)blockIdx.x >= p.nprod) {
      norm_epilogue<VD>(p, (int)blockIdx.x - p.nprod, (int)gridDim.x - p.nprod);
      return;
    }
  }

  // q/k tile addressing (element offsets): the swizzle of row r, the column of the row fragment for
  // key step s (lane row li, lane group g: keys 32s + 8g..+7), and the transposed K^T fragment of
  // state tile a = 2s + h against token rows 32u + 4g + m and 32u + 16 + 4g + m (ld8_tr_pair's
  // layout: lane 4m + q reads keys 32s + 8q + 4h..+3, i.e. chunk 4s + q, half h).
  auto kq_sw = [](int r) { return SWZ ? ((r & 7) << 1) : 0; };
  auto kq_col = [&](int s, int l_i, int l_g) { return (((4 * s + l_g) ^ kq_sw(l_i)) << 3); };
  // T - I and P tiles: 64 rows of 64 fp16 (128 B, unpadded), the 16-byte chunk c of row r at chunk
  // c ^ (r & 7). V and O slices: 64 rows of 32 bf16 (64 B), chunk c of row r at c ^ ((r >> 2) & 3).
  // Element offsets of (row r, column col); an access never spans two chunks.
  auto tp_off = [](int r, int col) { return r * kC + ((((col >> 3) ^ (r & 7)) << 3) | (col & 7)); };
  auto vo_off = [](int r, int col) { return r * kVB + ((((col >> 3) ^ ((r >> 2) & 3)) << 3) | (col & 7)); };
  auto kt_pair = [&](const f16* tile, int u, int a) {
    const int m = li >> 2, q = li & 3;
    const int row = 32 * u + 4 * g4 + m;  // row & 3 = m, (row >> 2) & 3 = g4: the swizzle of both rows
    const f16* p0 = tile + row * KP + ((((4 * (a >> 1) + q) ^ kq_sw(4 * g4 + m)) << 3) + 4 * (a & 1));
    const bf16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0));
    const bf16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p0 + 16 * KP));
    return __builtin_bit_cast(f16x8, bf16x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]});
  };

  // A_log and dt_bias are read per job (PERSIST) through the constant address space, as scalar loads:
  // as vector loads, the compiler follows each with a wait for every vector load in flight, which
  // drains the helpers' prefetched tiles.
  typedef const __attribute__((address_space(4))) float* const_f32p;
  // PERSIST: group gq of workgroups (blockIdx b on XCD b % 8 when the group count is a multiple of 8,
  // all NVB of a group on one XCD), its jobs and the chunks in all of them
  int gq = 0, gvb = 0;
  if constexpr (PERSIST) {
    if (p.nq % 8 == 0) {
      const int x = blockIdx.x % 8, j = blockIdx.x / 8;
      gq = 8 * (j / NVB) + x;
      gvb = j % NVB;
    } else {
      gq = blockIdx.x / NVB;
      gvb = blockIdx.x % NVB;
    }
  }
  // PERSIST: the group's job count and chunks in all its jobs (set by the prologue's scheduling)
  __shared__ int gjob[2];
  int njobs = 0, gsteps = 0;
  // a role's position in its chunk stream: chunk c of job j (PERSIST), with the job's tokens and heads
  struct Cursor {
    int j, c, nc, bos, eos, n, hv, h;
  };
  auto cur_job = [&](Cursor& u, int j) {
    u.j = j;
    u.c = 0;
    if (j < njobs) {
      // from the LDS copy (a scalar load here, whose result the role needs at once, stalled each
      // role for its latency at every job switch)
      const int4 e = jtab[j];
      u.bos = __builtin_amdgcn_readfirstlane(e.x);
      u.eos = __builtin_amdgcn_readfirstlane(e.y);
      u.n = __builtin_amdgcn_readfirstlane(e.z);
      u.hv = __builtin_amdgcn_readfirstlane(e.w);
      u.h = u.hv / (int)(p.HV / p.H);
      u.nc = (int)((u.eos - u.bos + kC - 1) / kC);
    } else {
      u.bos = u.eos = u.n = 0;
      u.hv = u.h = 0;
      u.nc = 0;
    }
  };
  auto cur_next = [&](Cursor& u) {
    if (++u.c >= u.nc && u.j < njobs) cur_job(u, u.j + 1);
  };
  const SliceLoc loc = PERSIST ? SliceLoc{gq, 0, 0, 0, 0, 0, gvb} : locate_slice<NVB>(p);
  const int64_t k_rank = loc.k, n = loc.n, bos = loc.bos, eos = loc.eos;
  const int hv = loc.hv, h = loc.h, vb = loc.vb;
  int nc = PERSIST ? 0 : (int)((eos - bos + kC - 1) / kC);
  const bool l2 = p.flags & GDN_FLAG_QK_L2NORM;
  const float a_log = p.A_log ? p.A_log[hv] : 0.f, dt_b = p.dt_bias ? p.dt_bias[hv] : 0.f;
  const bf16* __restrict__ qg = static_cast<const bf16*>(p.q);
  const bf16* __restrict__ kg = static_cast<const bf16*>(p.k);
  const bf16* __restrict__ vg = static_cast<const bf16*>(p.v);
  bf16* __restrict__ og = static_cast<bf16*>(p.o);

  auto chunk_len = [&](int c) {
    const int64_t c0 = bos + (int64_t)c * kC;
    return c < nc ? (int)((eos - c0) < kC ? (eos - c0) : kC) : 0;
  };
  // a chunk's first token, valid rows and heads: chunk c of the workgroup's sequence, or a cursor's chunk
  struct ChunkAt {
    int64_t c0;
    uint32_t len;
    int h, hv;
  };
  auto at = [&](int c) { return ChunkAt{bos + (int64_t)c * kC, (uint32_t)chunk_len(c), h, hv}; };
  auto cur_at = [&](const Cursor& u) {
    const int64_t c0 = u.bos + (int64_t)u.c * kC;
    return ChunkAt{c0, u.c < u.nc ? (uint32_t)((u.eos - c0) < kC ? (u.eos - c0) : kC) : 0u, u.h, u.hv};
  };

  // ------------------------------------------------------------------ helper-side staging
  // A helper issues the global loads of its tiles at the start of a chunk step and writes them to
  // LDS at the end of the same step, so the load registers are not live across the loop (sharing
  // loop-carried registers with the state waves' values would put register copies, and with them
  // waits for the loads, at the loop's join point). All loads go through buffer resources sized to
  // the chunk's valid rows: rows past the end (and chunks past the sequence) read as zeros.
  const uint32_t qk_row = (uint32_t)(p.H * KD * 2), v_row = (uint32_t)(p.HV * VD * 2), t_row = (uint32_t)(p.HV * kC * 2);
  const bool qk_wave = (w & 2) != 0;  // waves 2, 3, 6, 7
  // helper thread index of a lane value ln: 0..255 on the q/k waves, 0..127 on waves 4, 5
  auto thq_of = [&](int ln) { return (((w >> 2) << 1) | (w & 1)) * kWave + ln; };
  auto thv_of = [&](int ln) { return (w & 1) * kWave + ln; };
  const int thq = thq_of(lane), thv = thv_of(lane);
  constexpr int KSH = KS / 2;  // key steps of Y whose K fragments the state waves read ahead
  // The helpers' per-thread offsets are computed from `tq` (thq or thv of a lane id passed through
  // an empty asm inside the loop), so they are rebuilt in the helper branch each step instead of
  // being hoisted out of the loop into registers that would stay live through the state waves' code.
  // Thread tq of the q/k waves handles the 16-byte chunks tq + 256u of a q/k tile: row tq / KCH + u (256
  // / KCH), chunk tq % KCH.
  auto fetch_rows = [&](bf16x8 (&dst)[QKPT], const bf16* src, const ChunkAt& a, int tq) {
    const auto rs = make_rsrc(src + (a.c0 * p.H + a.h) * KD, a.len * qk_row);
    const uint32_t base = (uint32_t)(tq / KCH) * qk_row + (uint32_t)(tq % KCH) * 16;
#pragma unroll
    for (int u = 0; u < QKPT; ++u) dst[u] = buf_load16(rs, base + (uint32_t)(u * (256 / KCH)) * qk_row);
  };
  auto stage_rows = [&](const bf16x8 (&src)[QKPT], f16* dst, int tq) {  // bf16 rows (L2-normalised when asked) -> fp16
    f16* const d0 = dst + (tq / KCH) * KP + (((tq % KCH) ^ kq_sw(tq / KCH)) << 3);  // rows tq/KCH + 16u: same swizzle
#pragma unroll
    for (int u = 0; u < QKPT; ++u)
      *reinterpret_cast<f16x8*>(d0 + u * (256 / KCH) * KP) = bf16_to_f16x8(l2 ? l2norm_row_chunk<KCH>(src[u]) : src[u]);
  };
  // Thread tq of waves 4-5: T - I chunks tq + 128u (row tq / 8 + 16u, 8 chunks of 16 B per row)
  // and V-slice chunks tq + 128u (row tq / 4 + 32u, 4 chunks per row).
  auto fetch_tv = [&](bf16x8 (&pt)[4], bf16x8 (&pv)[2], const ChunkAt& a, int tq) {
    const int64_t c0 = a.c0;
    const uint32_t len = a.len;
    const int hv = a.hv;
    const auto rt = make_rsrc(p.tw + (c0 * p.HV + hv) * kC, len * t_row);
    const uint32_t bt = (uint32_t)(tq >> 3) * t_row + (uint32_t)(tq & 7) * 16;
#pragma unroll
    for (int u = 0; u < 4; ++u) pt[u] = buf_load16(rt, bt + (uint32_t)(16 * u) * t_row);
    const auto rv = make_rsrc(vg + (c0 * p.HV + hv) * VD + vb * kVB, len * v_row);
    const uint32_t bv = (uint32_t)(tq >> 2) * v_row + (uint32_t)(tq & 3) * 16;
#pragma unroll
    for (int u = 0; u < 2; ++u) pv[u] = buf_load16(rv, bv + (uint32_t)(32 * u) * v_row);
  };
  auto stage_tv = [&](const bf16x8 (&pt)[4], const bf16x8 (&pv)[2], int slot, int tq) {
    // rows tq / 8 + 16u (T) and tq / 4 + 32u (V) share their row's swizzle
    f16* const t0 = Tb[slot] + tp_off(tq >> 3, (tq & 7) * 8);
#pragma unroll
    for (int u = 0; u < 4; ++u) *reinterpret_cast<bf16x8*>(t0 + 16 * u * kC) = pt[u];  // fp16 bits, copied
    bf16* const v0 = Vc[slot] + vo_off(tq >> 2, (tq & 3) * 8);
#pragma unroll
    for (int u = 0; u < 2; ++u) *reinterpret_cast<bf16x8*>(v0 + 32 * u * kVB) = pv[u];
  };
  // The gate bits of a chunk are loaded by one 32-bit and one 16-bit load per tensor, both issued
  // whatever the dtype (a load whose width depends on the dtype would be two instructions on two
  // paths, and the loop-carried register they share would then be copied at the loop's join under
  // a wait for every load and store in flight). Each width has its own buffer resource: the one
  // matching the dtype spans exactly this head's elements of the chunk, from its first token to
  // the last byte of its last token, and the other spans zero bytes, so that load returns 0 and
  // touches no memory. (A 32-bit load at a 16-bit element would read 2 bytes beyond it, past the
  // end of the tensor for the last head of the last token.)
  struct GateBits {
    uint32_t g32, g16, b32, b16;
  };
  auto fetch_gates = [&](const ChunkAt& a, GateBits& r) {  // wave 4, lane = token
    const int64_t c0 = a.c0;
    const int hv = a.hv;
    const uint32_t eg = (uint32_t)dtype_bytes(p.dg), eb = (uint32_t)dtype_bytes(p.db);
    const uint32_t gb = (uint32_t)p.HV * eg, bb = (uint32_t)p.HV * eb;
    const uint32_t len = a.len;
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
  auto stage_gates = [&](int slot, const ChunkAt& a, const GateBits& r) {
    // (A_log through opaque_int: its exp is recomputed here, not held in a register)
    float al, db;
    if constexpr (PERSIST) {  // the job's head (scalar loads: read-only parameters)
      al = p.A_log ? reinterpret_cast<const_f32p>(reinterpret_cast<uint64_t>(p.A_log))[a.hv] : 0.f;
      db = p.dt_bias ? reinterpret_cast<const_f32p>(reinterpret_cast<uint64_t>(p.dt_bias))[a.hv] : 0.f;
    } else {
      al = __int_as_float(opaque_int(__float_as_int(a_log)));
      db = dt_b;
    }
    const uint32_t graw = p.dg == GDN_DTYPE_F32 ? r.g32 : r.g16, braw = p.db == GDN_DTYPE_F32 ? r.b32 : r.b16;
    chunk_gates_from_raw(gv[slot], graw, braw, p.dg, p.db, (int)a.len, p.flags, al, db, lane);
  };
  // waves 4-5: O of chunk c from Ob to HBM, rows tq / 4 + 32u; om keeps the stored values' magnitude maximum
  // O rows go out as non-temporal stores in the inference kernel: streamed past the caches, they
  // leave L2 to the q/k/T/V tiles that the slices of a chain share (config-1 call 130.3 -> 125.2 us,
  // same-box A/B). The training kernel keeps cached stores (non-temporal ones measured slower there).
  // With NORM they are also written through to memory (device scope), where the epilogue
  // workgroups, on any XCD, read them; or, when every epilogue workgroup of the chain runs on this
  // wave's XCD (o_local), they stay in that XCD's L2, where the workgroups read them.
  bool o_local = false;
  auto store_o = [&](int slot, const ChunkAt& a, int tq, u16x2& om) {
    const auto ro = make_rsrc(og + (a.c0 * p.HV + a.hv) * VD + vb * kVB, a.len * v_row);
    const int row = tq >> 2, c8 = tq & 3;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bf16x8 x = *reinterpret_cast<const bf16x8*>(&Ob[slot][vo_off(row + 32 * u, c8 * 8)]);
      om = bf16_mag_max(om, x);
      if (NORM && !o_local)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), ro,
                                               (int)((uint32_t)(row + 32 * u) * v_row + c8 * 16), 0,
                                               kPolSC1 | kPolNT);
      else
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), ro,
                                               (int)((uint32_t)(row + 32 * u) * v_row + c8 * 16), 0,
                                               SAVE ? 0 : NORM ? 0 : kPolNT);
    }
  };

  // NORM: the slice's progress word, the number of chunks whose O rows it has stored, written
  // through to memory once every storing thread has waited for those stores (s_waitcnt before a
  // barrier): an epilogue workgroup that reads the word with a device-scope load then sees the rows.
  auto publish_o = [&](int count) {
    const auto rp = make_rsrc(p.prog + (n * p.HV + hv) * kProgStride, NVB * 4);
    __builtin_amdgcn_raw_buffer_store_b32((unsigned)count, rp, vb * 4, 0, kPolSC1);
  };

  // scale * P^T of chunk c for key-row tiles JA..JA+JN-1 and query-row tiles TA..TA+TN-1 (tiles
  // with jt <= tt only): element (j = 16jt + 4g + r, t = 16tt + i), stored at Pb[t][tok_col(j)].
  // Waves 2, 3, 6, 7 (SIMDs 2 and 3) take the 2x2, 2x2, 2x1 and 2x1 tile blocks of the lower triangle.
  auto p_job = [&](auto ja_c, auto jn_c, auto ta_c, auto tn_c, int c, int ln) {
    const int li = ln & 15, g4 = ln >> 4;
    constexpr int JA = decltype(ja_c)::value, JN = decltype(jn_c)::value;
    constexpr int TA = decltype(ta_c)::value, TN = decltype(tn_c)::value;
    const f16* kb = Kc[c % 3];
    const f16* qb = Qc[c & 1];
    f16* pw = Pb[c & 1];
    const ChunkGates& gs = gv[c % 3];
    f32x4 acc[JN][TN];
#pragma unroll
    for (int a = 0; a < JN; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{};
    // every fragment and gate read of the job first, then the MFMAs: one LDS round trip instead of
    // one per key step
    f16x8 fk[KS][JN], fq[KS][TN];
    float gtv[TN];
    float4 gjv4[JN];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int a = 0; a < JN; ++a) fk[s][a] = ld8h(kb + (16 * (JA + a) + li) * KP + kq_col(s, li, g4));
#pragma unroll
      for (int b = 0; b < TN; ++b) fq[s][b] = ld8h(qb + (16 * (TA + b) + li) * KP + kq_col(s, li, g4));
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) gtv[b] = gs.gam[16 * (TA + b) + li];
#pragma unroll
    for (int a = 0; a < JN; ++a) gjv4[a] = ld4f(&gs.gam[16 * (JA + a) + 4 * g4]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int a = 0; a < JN; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          if (JA + a <= TA + b) acc[a][b] = mmah(fk[s][a], fq[s][b], acc[a][b]);
#pragma unroll
    for (int a = 0; a < JN; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) {
        const int jt = JA + a, tt_ = TA + b;
        if (jt > tt_) continue;
        const int tt = 16 * tt_ + li, j0 = 16 * jt + 4 * g4;
        const float gt = gtv[b];
        const float4 gj = gjv4[a];
        const float gjv[4] = {gj.x, gj.y, gj.z, gj.w};
        float val[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) val[r] = (jt < tt_ || j0 + r <= tt) ? p.scale * __expf(gt - gjv[r]) * acc[a][b][r] : 0.f;
        *reinterpret_cast<f16x4*>(pw + tp_off(tt, tok_col(j0))) = to_f16x4(val[0], val[1], val[2], val[3]);
      }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  auto run_p_side = [&](int c, int ln) {
    switch (w) {
      case 2: p_job(I0{}, I2{}, I0{}, I2{}, c, ln); break;   // (0,0) (0,1) (1,1)
      case 3: p_job(I2{}, I2{}, I2{}, I2{}, c, ln); break;   // (2,2) (2,3) (3,3)
      case 6: p_job(I0{}, I2{}, I2{}, I1{}, c, ln); break;   // (0,2) (1,2)
      case 7: p_job(I0{}, I2{}, I3{}, I1{}, c, ln); break;   // (0,3) (1,3)
      default: break;
    }
  };

  // ------------------------------------------------------------------ state-side registers
  const int sw = w & 1;  // state wave 0 or 1: value columns 16 sw .. 16 sw + 15 of the slice
  // Loop-carried: S tiles; Z^T = S^T Q^T of the current chunk, tile tb (value column 4g + r, token
  // 16tb + i); (S_2s, S_2s+1) in fp16 (SB); Y = K S of the chunk the next step processes (YN,
  // computed at the end of a step: its K was staged a step earlier, so it needs no barrier).
  f32x4 S[KT], Zt[4], SB[KS], YN[4];
  float ec_next = 1.f;  // e^{gam_c} of the chunk the next step processes
  auto sb = [&](int s) { return __builtin_bit_cast(f16x8, SB[s]); };
  const int64_t sbase = (n * p.HV + hv) * (int64_t)KD * VD + vb * kVB + 16 * sw;
  // SAVE: global index of the sequence's first chunk (chunks before it with cu_seqlens)
  const int64_t cg_first = SAVE ? (p.cu ? (int64_t)p.chunk_first[n] : n * ((p.T + kC - 1) / kC)) : 0;
  auto make_sb = [&]() {
#pragma unroll
    for (int s = 0; s < KS; ++s) SB[s] = __builtin_bit_cast(f32x4, pack8h(S[2 * s], S[2 * s + 1]));
  };
  // SAVE: S (the state entering chunk c) as bf16 into its [V][K] slot: a buffer resource over the
  // chunk-head's state (uniform base), lane offsets from an opaque lane id
  auto save_state = [&](int c) {
    const auto rs = make_rsrc(p.hs + ((cg_first + c) * p.HV + hv) * (int64_t)(KD * VD), (uint32_t)(KD * VD * 2));
    const int ls = opaque_int(lane);
    const uint32_t off = (uint32_t)(((vb * kVB + 16 * sw + (ls & 15)) * KD + 8 * (ls >> 4)) * 2);
#pragma unroll
    for (int a = 0; a < KT; ++a)
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, to_bf16x4(S[a][0], S[a][1], S[a][2], S[a][3])), rs,
                                            (int)(off + (32 * (a >> 1) + 4 * (a & 1)) * 2), 0, 0);
  };
  // Each phase of the state step issues the LDS reads of the next phase before its own MFMAs, and
  // the scheduler may not move instructions across the phase boundaries: LDS reads complete in
  // order, so every phase finds its operands arrived or in flight instead of starting a round trip.
  auto phase = [] { __builtin_amdgcn_sched_barrier(0); };

  GateBits ngate{0, 0, 0, 0};  // wave 4: raw gate bits of the chunk two steps ahead, in flight

  // ------------------------------------------------------------------ prologue
  if (t == 0) {
    bad = 0;
    first_bad = 0x7fffffff;
  }
  if constexpr (PERSIST) {
    schedule_group(p, gq, jtab, gjob, sched);
    njobs = gjob[0];
    gsteps = gjob[1];
    nc = gsteps;
  }
  // P is causally lower: its tiles above the diagonal stay zero for the whole run
  for (int e = t; e < kC * kC / 8; e += kNT) {
    reinterpret_cast<f16x8*>(Pb[0])[e] = f16x8{};
    reinterpret_cast<f16x8*>(Pb[1])[e] = f16x8{};
  }
  // Each role runs its own prologue and chunk loop; every loop runs nc steps with one barrier each,
  // so the barriers line up. Separate loops keep each role's loop-carried registers out of the
  // others' register allocation: the helpers hold the global loads of the next step's tiles across
  // the barrier, a full step of latency hiding.
  if (w < 2) {
    // PERSIST: the job of the current step (no initial state: every job starts from zero)
    Cursor sc{};
    if constexpr (PERSIST) cur_job(sc, 0);
#pragma unroll
    for (int a = 0; a < KT; ++a) {
      const int kd0 = 32 * (a >> 1) + 8 * g4 + 4 * (a & 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) S[a][r] = !PERSIST && p.h0 ? p.h0[sbase + (int64_t)(kd0 + r) * VD + li] : 0.f;
    }
    make_sb();
    if constexpr (SAVE) {
      if (nc > 0) save_state(0);
    }
    __syncthreads();
    if (nc > 0) {
      f16x8 qf[KS][4];
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) qf[s2][tb] = ld8h(Qc[0] + (16 * tb + li) * KP + kq_col(s2, li, g4));
      ec_next = __expf(gv[0].gam[kC - 1]);
      // Y = K S of chunk 0 (the steps compute the next chunk's Y at their end)
#pragma unroll
      for (int b = 0; b < 4; ++b) YN[b] = f32x4{};
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2) {
        f16x8 kf0[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) kf0[b] = ld8h(Kc[0] + (16 * b + li) * KP + kq_col(s2, li, g4));
#pragma unroll
        for (int b = 0; b < 4; ++b) YN[b] = mmah(kf0[b], sb(s2), YN[b]);
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) Zt[tb] = f32x4{};
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) Zt[tb] = mmah(sb(s2), qf[s2][tb], Zt[tb]);
    }
    __syncthreads();
    // Slots in use during step i: state waves read K_i, T_i, V_i, P_i, gates_i and Q_{i+1}, write
    // O_i; helpers read K_{i+1}, Q_{i+1}, gates_{i+1} (P_{i+1}) and O_{i-1}, write K_{i+2}, Q_{i+2},
    // T_{i+1}, V_{i+1}, P_{i+1}, gates_{i+2}. No slot is written and read in the same step.
    auto step = [&](auto ph_c, int i) {
      constexpr int PH = decltype(ph_c)::value;
      const f16* kb = Kc[PH % 3];
      const f16* tp = Tb[PH & 1];
      const bf16* vp = Vc[PH & 1];
      const f16* pp = Pb[PH & 1];
      bf16* op = Ob[PH & 1];
      const ChunkGates& G = gv[PH % 3];

      // The chain S -> Y -> X -> Delta -> Delta~ -> S' runs through phases 6 (Y of the next chunk,
      // from S' in fp16) and 1-5; the rest is placed where it overlaps the chain: the e^{gam_c}
      // scaling of S under the phase-1 reads, and O of this chunk with Z^T of the next in phase 6,
      // between the two halves of the next Y. Phases 5 and 6 run unconditionally: after the last
      // chunk they read slots holding stale tiles and compute values nobody uses, which keeps the
      // step free of branches (a branch around loads costs the register allocator dearly here).
      // Computing the next Y before the barrier instead of after it took ~2.5 us off a config-1
      // call (same-box A/B, bitwise-equal outputs).
      // ---- 1: reads for X (V, beta, beta e^gam); S *= e^{gam_c} (Y used S in fp16)
      bf16x4 vv[4];
      float4 bt[4], bg[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        vv[b] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(  // ld4_tr's lanes on the swizzled slice
            (lds_bf16x4*)(vp + vo_off(16 * b + 4 * g4 + (li >> 2), 16 * sw + 4 * (li & 3))));
        bt[b] = ld4f(&G.bet[16 * b + 4 * g4]);
        bg[b] = ld4f(&G.begam[16 * b + 4 * g4]);
      }
      const float ec = ec_next;
      phase();
      f32x4 D[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) D[b] = YN[b];  // Y = K S of this chunk, computed at the previous step's end
#pragma unroll
      for (int a = 0; a < KT; ++a) S[a] *= ec;
      phase();
      // ---- 2: reads of T - I; X = beta V - beta e^gam Y (kept in fp32 as the Delta accumulator's start)
      f16x8 tf[6];
      tf[0] = ld8h(tp + tp_off(0 + li, 0 + 8 * g4));
      tf[1] = ld8h(tp + tp_off(16 + li, 0 + 8 * g4));
      tf[2] = ld8h(tp + tp_off(32 + li, 0 + 8 * g4));
      tf[3] = ld8h(tp + tp_off(48 + li, 0 + 8 * g4));
      tf[4] = ld8h(tp + tp_off(32 + li, 32 + 8 * g4));
      tf[5] = ld8h(tp + tp_off(48 + li, 32 + 8 * g4));
      phase();
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        D[b][0] = bt[b].x * (float)vv[b][0] - bg[b].x * D[b][0];
        D[b][1] = bt[b].y * (float)vv[b][1] - bg[b].y * D[b][1];
        D[b][2] = bt[b].z * (float)vv[b][2] - bg[b].z * D[b][2];
        D[b][3] = bt[b].w * (float)vv[b][3] - bg[b].w * D[b][3];
      }
      const f16x8 xb0 = pack8h(D[0], D[1]), xb1 = pack8h(D[2], D[3]);
      phase();
      // ---- 3: reads of e^{gam_c - gam} and of K^T for the first half of the state tiles;
      //      Delta = X + (T - I) X (T - I vanishes above the diagonal); Delta~ = e^{gam_c - gam} Delta
      constexpr int KH = KT / 2;
      float4 dla[2], dlb[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        dla[u] = ld4f(&G.dlast[32 * u + 4 * g4]);
        dlb[u] = ld4f(&G.dlast[32 * u + 16 + 4 * g4]);
      }
      f16x8 ktf[KT][2];
#pragma unroll
      for (int a = 0; a < KH; ++a)
#pragma unroll
        for (int u = 0; u < 2; ++u) ktf[a][u] = kt_pair(kb, u, a);
      phase();
      D[0] = mmah(tf[0], xb0, D[0]);
      D[1] = mmah(tf[1], xb0, D[1]);
      D[2] = mmah(tf[2], xb0, D[2]);
      D[3] = mmah(tf[3], xb0, D[3]);
      D[2] = mmah(tf[4], xb1, D[2]);
      D[3] = mmah(tf[5], xb1, D[3]);
      f16x8 dt[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f32x4 x0 = {dla[u].x * D[2 * u][0], dla[u].y * D[2 * u][1], dla[u].z * D[2 * u][2], dla[u].w * D[2 * u][3]};
        const f32x4 x1 = {dlb[u].x * D[2 * u + 1][0], dlb[u].y * D[2 * u + 1][1], dlb[u].z * D[2 * u + 1][2],
                          dlb[u].w * D[2 * u + 1][3]};
        dt[u] = pack8h(x0, x1);
      }
      const f16x8 db0 = pack8h(D[0], D[1]), db1 = pack8h(D[2], D[3]);
      phase();
      // ---- 4: K^T reads for the second half, P and scale e^gam reads; S' = e^{gam_c} S + K^T Delta~
#pragma unroll
      for (int a = KH; a < KT; ++a)
#pragma unroll
        for (int u = 0; u < 2; ++u) ktf[a][u] = kt_pair(kb, u, a);
      f16x8 pf[6];
      float eg[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) pf[tb] = ld8h(pp + tp_off(16 * tb + li, 8 * g4));
      pf[4] = ld8h(pp + tp_off(32 + li, 32 + 8 * g4));
      pf[5] = ld8h(pp + tp_off(48 + li, 32 + 8 * g4));
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) eg[tb] = p.scale * G.egam[16 * tb + li];
      phase();
#pragma unroll
      for (int a = 0; a < KT; ++a)
#pragma unroll
        for (int u = 0; u < 2; ++u) S[a] = mmah(ktf[a][u], dt[u], S[a]);
      phase();
      if constexpr (PERSIST) {
        // the last chunk of a job: the next job starts from the zero state
        if (sc.c + 1 >= sc.nc) {
#pragma unroll
          for (int a = 0; a < KT; ++a) S[a] = f32x4{};
        }
        cur_next(sc);
      }
      // ---- 5: Q reads and the first half of the K reads of the next chunk; S in fp16
      const f16* kn = Kc[(PH + 1) % 3];
      f16x8 kfa[KSH][4];
#pragma unroll
      for (int s2 = 0; s2 < KSH; ++s2)
#pragma unroll
        for (int b = 0; b < 4; ++b) kfa[s2][b] = ld8h(kn + (16 * b + li) * KP + kq_col(s2, li, g4));
      f16x8 qf[KS][4];
      {
        const f16* qb = Qc[(PH + 1) & 1];
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) qf[s2][tb] = ld8h(qb + (16 * tb + li) * KP + kq_col(s2, li, g4));
      }
      make_sb();
      phase();
      // ---- 6: the next chunk's Y (first half), its e^{gam_c}; O^T = scale e^gam Z^T + Delta^T (scale P)^T
      //      -> Ob[token][column]; K reads of Y's second half; Z^T = S^T Q^T of the next chunk; Y's
      //      second half
      ec_next = __expf(gv[(PH + 1) % 3].gam[kC - 1]);
      phase();
      // the next chunk's Y = K S from S' in fp16 (its K was staged a step ago): first half
#pragma unroll
      for (int b = 0; b < 4; ++b) YN[b] = f32x4{};
#pragma unroll
      for (int s2 = 0; s2 < KSH; ++s2)
#pragma unroll
        for (int b = 0; b < 4; ++b) YN[b] = mmah(kfa[s2][b], sb(s2), YN[b]);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 o = Zt[tb] * eg[tb];
        o = mmah(db0, pf[tb], o);
        if (tb >= 2) o = mmah(db1, pf[tb + 2], o);
        const bf16x4 ob = to_bf16x4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<bf16x4*>(op + vo_off(16 * tb + li, 16 * sw + 4 * g4)) = ob;
      }
      f16x8 kfb[KS - KSH][4];
#pragma unroll
      for (int s2 = KSH; s2 < KS; ++s2)
#pragma unroll
        for (int b = 0; b < 4; ++b) kfb[s2 - KSH][b] = ld8h(kn + (16 * b + li) * KP + kq_col(s2, li, g4));
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) Zt[tb] = f32x4{};
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) Zt[tb] = mmah(sb(s2), qf[s2][tb], Zt[tb]);
#pragma unroll
      for (int s2 = KSH; s2 < KS; ++s2)
#pragma unroll
        for (int b = 0; b < 4; ++b) YN[b] = mmah(kfb[s2 - KSH][b], sb(s2), YN[b]);
      if constexpr (SAVE) {
        // S' (updated in phase 4) is the state entering chunk i + 1; stored at the step's end, away
        // from the helpers' load burst at its start
        if (i + 1 < nc) save_state(i + 1);
      }
      __syncthreads();
    };
    // unrolled by 6 so that every slot index (mod 2 and mod 3) is a constant
    for (int i = 0; i < nc; i += 6) {
      step(std::integral_constant<int, 0>{}, i);
      if (i + 1 < nc) step(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < nc) step(std::integral_constant<int, 2>{}, i + 2);
      if (i + 3 < nc) step(std::integral_constant<int, 3>{}, i + 3);
      if (i + 4 < nc) step(std::integral_constant<int, 4>{}, i + 4);
      if (i + 5 < nc) step(std::integral_constant<int, 5>{}, i + 5);
    }
    if (!PERSIST && p.ht) {  // (PERSIST: stored at each job's last chunk)
      uint32_t smax = 0;  // magnitude bits: at or above 0x7f800000 for inf and NaN
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kd0 = 32 * (a >> 1) + 8 * g4 + 4 * (a & 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p.ht[sbase + (int64_t)(kd0 + r) * VD + li] = S[a][r];
          smax = max(smax, __float_as_uint(S[a][r]) & 0x7fffffffu);
        }
      }
      if (smax >= 0x7f800000u) __hip_atomic_fetch_or(&bad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  } else if (qk_wave) {
    // the chunk stream's q/k loads in order: chunk c of the sequence, or the cursor's next chunk
    Cursor fq{};
    if constexpr (PERSIST) cur_job(fq, 0);
    auto qk_src = [&](int c) {
      if constexpr (PERSIST) {
        const ChunkAt a = cur_at(fq);
        cur_next(fq);
        return a;
      } else {
        return at(c);
      }
    };
    // K/Q of chunks 0 and 1 staged, chunk 2 in flight
    bf16x8 pk[QKPT], pq[QKPT];
    for (int c = 0; c < 2; ++c) {
      const ChunkAt a = qk_src(c);
      fetch_rows(pk, kg, a, thq);
      fetch_rows(pq, qg, a, thq);
      stage_rows(pk, Kc[c], thq);
      stage_rows(pq, Qc[c], thq);
    }
    {
      const ChunkAt a = qk_src(2);
      fetch_rows(pk, kg, a, thq);
      fetch_rows(pq, qg, a, thq);
    }
    __syncthreads();
    if (nc > 0) run_p_side(0, lane);
    __syncthreads();
    // K/Q of chunk i+2 (loaded a step ago) into LDS, the loads of chunk i+3, then P of chunk i+1:
    // the loads go out before P. Measured per config-1 call against this order (same box): P,
    // staging, loads +3 us; staging, P, loads +10 us.
    for (int i = 0; i < nc; ++i) {
      const int tq = thq_of(opaque_int(lane));
      stage_rows(pk, Kc[(i + 2) % 3], tq);
      stage_rows(pq, Qc[i & 1], tq);
      const ChunkAt a = qk_src(i + 3);
      fetch_rows(pk, kg, a, tq);
      fetch_rows(pq, qg, a, tq);
      if (i + 1 < nc) run_p_side(i + 1, opaque_int(lane));
      __syncthreads();
    }
  } else {
    // the chunk streams of this role, each walked in order: T/V loads and gate staging (the same
    // chunks), gate loads (wave 4), O stores
    Cursor ct{}, cgf{}, co{};
    if constexpr (PERSIST) {
      cur_job(ct, 0);
      cur_job(cgf, 0);
      cur_job(co, 0);
    }
    auto src = [&](Cursor& u, int c) {
      if constexpr (PERSIST) {
        const ChunkAt a = cur_at(u);
        cur_next(u);
        return a;
      } else {
        return at(c);
      }
    };
    // T/V of chunk 0 staged and chunk 1 in flight; gates of chunks 0 and 1 staged, chunk 2 in flight
    bf16x8 pt[4], pv[2];
    u16x2 om = {0, 0};
    const ChunkAt a0 = src(ct, 0), a1 = src(ct, 1);
    fetch_tv(pt, pv, a0, thv);
    stage_tv(pt, pv, 0, thv);
    fetch_tv(pt, pv, a1, thv);
    if (w == 4) {
      for (int c = 0; c < 2; ++c) {
        GateBits gb0;
        fetch_gates(src(cgf, c), gb0);
        stage_gates(c, c ? a1 : a0, gb0);
      }
      fetch_gates(src(cgf, 2), ngate);
    }
    __syncthreads();
    __syncthreads();
    unsigned posted = 0;  // NORM: lane l, the XCC id (+ 1) epilogue workgroup l of the chain posted
    for (int i = 0; i < nc; ++i) {  // gates of chunk i+2, O of chunk i-1 out, T/V of chunk i+1 into LDS, loads of chunk i+2
      if constexpr (NORM) {
        // the epilogue workgroups' posts, read in step 0 and checked in step 1, before the first O
        // store (each wave decides for its own stores)
        if (i <= 1) {
          const auto rb = make_rsrc(p.prog + (n * p.HV + hv) * kProgStride, kProgStride * 4);
          if (i == 0) {
            posted = __builtin_amdgcn_raw_buffer_load_b32(rb, (kEpiPostBase + lane) * 4, 0, kPolSC1);
          } else {
            const int64_t nr = ((int64_t)gridDim.x - p.nprod) / (p.N * p.HV);
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            o_local = nr <= kEpiPostMax && __builtin_amdgcn_ballot_w64(lane < nr && posted != wave_xcc() + 1) == 0;
          }
        }
        // this thread's O stores of chunk i - 2 (issued last step, with the loads this step stages)
        // have completed; every storing thread's stores of chunk i - 3 completed before the
        // previous step's barrier, so chunks 0 .. i - 3 are published
        // (never past a chunk whose O held an inf or NaN: the recomputation below rewrites those)
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        if (w == 5 && lane == 0 && i >= 3) publish_o(min(i - 2, first_bad));
      }
      const int tq = thv_of(opaque_int(lane));
      const ChunkAt a2 = src(ct, i + 2);  // the chunk whose gates are staged and T/V loaded this step
      if (w == 4) {  // gates of chunk i+2 (loaded a step ago), then the loads for chunk i+3
        stage_gates((i + 2) % 3, a2, ngate);
        fetch_gates(src(cgf, i + 3), ngate);
      }
      if (i > 0) {
        store_o((i - 1) & 1, src(co, i - 1), tq, om);
        if constexpr (NORM) {
          if (om[0] >= 0x7f80 || om[1] >= 0x7f80) atomicMin(&first_bad, i - 1);
        }
      }
      stage_tv(pt, pv, (i + 1) & 1, tq);
      fetch_tv(pt, pv, a2, tq);
      __syncthreads();
    }
    if (nc > 0) store_o((nc - 1) & 1, src(co, nc - 1), thv, om);
    if constexpr (NORM) {
      if (om[0] >= 0x7f80 || om[1] >= 0x7f80) atomicMin(&first_bad, nc - 1);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);  // before the barrier ahead of the last word
    }
    if (om[0] >= 0x7f80 || om[1] >= 0x7f80) __hip_atomic_fetch_or(&bad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }

  // ------------------------------------------------------------------ recovery
  // A slice whose fp16 matrix-core operands left the fp16 range (65504) -- for instance from inputs
  // of a scale fp32 and bf16 hold but fp16 does not -- has stored an inf or NaN in O or the final
  // state. The slice then computes its 32 columns again by the fp32 token-by-token recurrence
  // (value columns of the state evolve independently), overwriting O, the final state and (SAVE)
  // the saved chunk states, and flags the call only if that recomputation is non-finite as well
  // (non-finite inputs). Slices that stored finite values skip it: the cost is this barrier.
  // With NORM the slice has published no chunk from the first one whose O was not finite: the
  // recomputation rewrites O from that chunk on (the epilogue workgroups may already have
  // normalised the chunks before it in place), writes it back to memory (an agent-scope release)
  // and then publishes every chunk.
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(bad)) {
    if constexpr (NORM) {
      const int fb = first_bad;
      const ChunkParams pr = reload_params();
      const SliceLoc lr = locate_slice<NVB>(pr);
      recover_slice<KD, VD, false>(pr, lr.n, lr.hv, lr.h, lr.vb, lr.bos, lr.eos, 0, (bf16*)&Kc[0][0],
                                   (bf16*)&Qc[0][0], (bf16*)&Vc[0][0], &gv[0], fb);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __syncthreads();
    } else {
      const ChunkParams pr = reload_params();
      if constexpr (PERSIST) {
        // every job of the group, in turn (the workgroup's V-slice of each)
        // (the job list is still in LDS: the recomputation stages its tiles in the chunk slots)
        const int rvb = pr.nq % 8 == 0 ? (int)((blockIdx.x / 8) % NVB) : (int)(blockIdx.x % NVB);
        const int rjobs = gjob[0];
        for (int j = 0; j < rjobs; ++j) {
          const int4 e = jtab[j];
          recover_slice<KD, VD, SAVE>(pr, e.z, e.w, e.w / (int)(pr.HV / pr.H), rvb, e.x, e.y, 0, (bf16*)&Kc[0][0],
                                      (bf16*)&Qc[0][0], (bf16*)&Vc[0][0], &gv[0]);
          __syncthreads();  // the next job's staging reuses the tiles
        }
      } else {
        const SliceLoc lr = locate_slice<NVB>(pr);
        const int64_t cgr = SAVE ? (pr.cu ? (int64_t)pr.chunk_first[lr.n] : lr.n * ((pr.T + kC - 1) / kC)) : 0;
        recover_slice<KD, VD, SAVE>(pr, lr.n, lr.hv, lr.h, lr.vb, lr.bos, lr.eos, cgr, (bf16*)&Kc[0][0],
                                    (bf16*)&Qc[0][0], (bf16*)&Vc[0][0], &gv[0]);
      }
    }
  }
  if constexpr (NORM) {
    if (t == 5 * kWave) publish_o(nc);
  }
}

}  // namespace gdn

using namespace gdn;

// Workspace layouts: the two-kernel prefill keeps the T - I rows first, then the varlen index; the
// cooperative prefill keeps its package ring and sync words first, then the varlen index. The size
// covers the ring only while SORERNN_PREFILL=coop selects that route: the ring is 8 slots of 47 KB per
// (sequence, value head), which for many short sequences dwarfs the two-kernel prefill's 128 bytes per
// token-head (6 GB against 0.2 GB for 1,000 sequences of 100 tokens at 16 heads).
namespace {
size_t index_bytes(int64_t N, int varlen) {
  return varlen ? (size_t)(align256((N + 1) * 4) + align256(N * 4)) : 0;
}
size_t coop_front_bytes(int64_t T, int64_t HV, int64_t N) {
  return (size_t)(coop_ring_bytes(N * HV, T) + coop_sync_bytes(N * HV));
}
// The cooperative single-launch prefill, selected per call with SORERNN_PREFILL=coop.
bool coop_selected() {
  const char* const sel = getenv("SORERNN_PREFILL");
  return sel && !strcmp(sel, "coop");
}
}  // namespace

extern "C" size_t gdn_chunk_workspace_size(int64_t B, int64_t T, int64_t HV, int64_t N, int varlen) {
  if (B <= 0 || T < 0 || HV <= 0 || N <= 0) return 0;
  size_t front = (size_t)chunk_t_bytes(B * T, HV);
  if (coop_selected()) front = std::max(front, coop_front_bytes(T, HV, N));
  return front + index_bytes(N, varlen);
}

namespace {

constexpr int kMaxDevices = 64;

// Non-finite output flags, one device-accessible word per device (null: no check); written under
// g_flag_mu, read without it by every launch.
std::mutex g_flag_mu;
std::atomic<unsigned*> g_range_flag[kMaxDevices] = {};

// The device that runs `stream` (the current device for the null stream), or -1.
int stream_device(hipStream_t stream) {
  int dev = -1;
  if (stream ? hipStreamGetDevice(stream, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) return -1;
  return dev;
}

// The fused norm's progress words (after the chunk workspace): one per chain and V / 32 slice, in a
// 256-byte block per chain.
size_t norm_prog_bytes(int64_t N, int64_t HV, int64_t V) {
  static_assert(128 / kVB <= kProgStride, "a chain's words fit its block");
  (void)V;
  return (size_t)align256(N * HV * kProgStride * 4);
}

int chunk_fwd_impl(const void* q, const void* k, const void* v, const void* g, const void* beta,
                   const float* initial_state, void* o, float* final_state, const void* cu_seqlens, int64_t B,
                   int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N, int qkv_dtype, int g_dtype,
                   int beta_dtype, float scale, unsigned flags, const float* A_log, const float* dt_bias,
                   void* chunk_states, void* workspace, size_t workspace_bytes, void* stream,
                   const void* ngate = nullptr, const float* nweight = nullptr, float neps = 0.f, int nsplit = 0) {
  if (!q || !k || !v || !g || !beta || !o) {
    gdn_internal_set_error("gdn_chunk_fwd: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  if (B <= 0 || T < 0 || H <= 0 || HV <= 0 || HV % H || N <= 0) {
    gdn_internal_set_error("gdn_chunk_fwd: bad sizes B=%lld T=%lld H=%lld HV=%lld N=%lld", (long long)B, (long long)T,
                           (long long)H, (long long)HV, (long long)N);
    return GDN_ERR_INVALID;
  }
  if (cu_seqlens ? B != 1 : N != B) {
    gdn_internal_set_error("gdn_chunk_fwd: cu_seqlens requires B == 1 (and N == B without it)");
    return GDN_ERR_INVALID;
  }
  if ((flags & GDN_FLAG_GATE_IN_KERNEL) && (!A_log || !dt_bias)) {
    gdn_internal_set_error("gdn_chunk_fwd: gate in kernel needs A_log and dt_bias");
    return GDN_ERR_INVALID;
  }
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) {
    gdn_internal_set_error("gdn_chunk_fwd: head dims K=%lld V=%lld unsupported (each must be 64 or 128)", (long long)K,
                           (long long)V);
    return GDN_ERR_UNSUPPORTED;
  }
  if (qkv_dtype != GDN_DTYPE_BF16) {
    gdn_internal_set_error("gdn_chunk_fwd: q/k/v dtype %d unsupported by the chunk kernel (bf16 only)", qkv_dtype);
    return GDN_ERR_UNSUPPORTED;
  }
  const bool norm = ngate != nullptr;
  if (norm && (!nweight || chunk_states)) {
    gdn_internal_set_error("gdn_chunk_fwd_gated_norm: the norm weight is required (inference calls only)");
    return GDN_ERR_INVALID;
  }
  const size_t base_need = gdn_chunk_workspace_size(B, T, HV, N, cu_seqlens != nullptr);
  const size_t need = norm && base_need ? base_need + norm_prog_bytes(N, HV, V) : base_need;
  if (need > 0 && (!workspace || workspace_bytes < need)) {
    gdn_internal_set_error("gdn_chunk_fwd: workspace of %zu bytes needed (got %zu)", need,
                           workspace ? workspace_bytes : (size_t)0);
    return GDN_ERR_INVALID;
  }
  if (T == 0) return GDN_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int cu_i32 = (flags & GDN_FLAG_CU_INT32) ? 1 : 0;
  const int dev = stream_device(s);
  unsigned* const range_flag = dev >= 0 && dev < kMaxDevices ? g_range_flag[dev].load(std::memory_order_acquire)
                                                             : nullptr;
  // The cooperative single-launch prefill for K = V = 128 inference calls, selected per call with
  // SORERNN_PREFILL=coop (the two-kernel prefill otherwise, which is faster at every measured size).
  // The workspace check above used the size that includes its ring when it is selected.
  if (!chunk_states && !norm && K == 128 && V == 128 && coop_selected()) {
    char* const ws = static_cast<char*>(workspace);
    const int64_t chains = N * HV;
    const size_t front = coop_front_bytes(T, HV, N);
    int* const chunk_first = cu_seqlens ? reinterpret_cast<int*>(ws + front) : nullptr;
    int* const order = cu_seqlens ? reinterpret_cast<int*>(ws + front + align256((N + 1) * 4)) : nullptr;
    if (cu_seqlens) {
      const int rc = launch_chunk_index(cu_seqlens, cu_i32, N, chunk_first, order, s);
      if (rc != GDN_OK) return rc;
    }
    unsigned* const sync = reinterpret_cast<unsigned*>(ws + coop_ring_bytes(chains, T));
    CoopArgs a{q, k, v, g, beta, initial_state, o, final_state, cu_seqlens, order, cu_i32, T, H, HV, N,
               g_dtype, beta_dtype, scale, flags, A_log, dt_bias, ws, sync, range_flag, nullptr};
    return launch_chunk_coop(a, s);
  }
  const int64_t nvb = V / kVB;
  int64_t blocks = N * HV * nvb;
  if (blocks > 0x7fffffff) {
    gdn_internal_set_error("gdn_chunk_fwd: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  // The persistent grid for inference calls with cu_seqlens and no initial or final state whose
  // chains (sequence, value head) are many against the machine: one workgroup per CU, in groups of V / 32 (one per V-slice), each
  // group walking a job list of at least four chains on average (snake order over the chains sorted
  // longest first, so the lists' lengths come out even). Fewer, longer chains keep one workgroup per
  // slice, dispatched longest first: there the longest sequence sets the time.
  const int64_t cus = device_compute_units(s);
  const int64_t nq = cus / nvb;
  // The fused norm runs in epilogue workgroups of the same launch when the chains' slices leave at
  // least two CUs per chain free (one workgroup per CU, so the whole grid is resident at once;
  // config 4's 32 chains have 128 slices and 128 epilogue workgroups on 256 CUs). Otherwise the
  // chunk kernel stores O into the output and the norm kernel follows in place.
  const bool epi = norm && blocks + 2 * N * HV <= cus;
  const bool persist = cu_seqlens && !chunk_states && !epi && !initial_state && !final_state && N <= kOrderMax &&
                       nq >= 1 && N * HV >= 4 * nq && (N * HV + nq - 1) / nq <= kJobTab;
  f16* tw = static_cast<f16*>(workspace);
  char* const ws = static_cast<char*>(workspace);
  const int* chunk_first = cu_seqlens ? reinterpret_cast<const int*>(ws + chunk_t_bytes(B * T, HV)) : nullptr;
  const int* order =
      cu_seqlens ? reinterpret_cast<const int*>(ws + chunk_t_bytes(B * T, HV) + align256((N + 1) * 4)) : nullptr;
  ChunkPrepParams pp{k, g, beta, tw, cu_seqlens, chunk_first, order, cu_i32, T, H, HV, N, g_dtype, beta_dtype, flags,
                     A_log, dt_bias};
  const int rc = launch_chunk_prep(pp, B, K, s);
  if (rc != GDN_OK) return rc;
  ChunkParams p{q, k, v, g, beta, initial_state, o, final_state, tw, cu_seqlens, order, cu_i32, T, H, HV, N,
                g_dtype, beta_dtype, scale, flags, A_log, dt_bias, static_cast<bf16*>(chunk_states), chunk_first,
                range_flag, static_cast<const bf16*>(ngate), nweight, neps, nsplit, nullptr};
  if (persist) {
    p.nq = (int)nq;
    blocks = nq * nvb;
  }
  if (epi) {
    p.nprod = (int)blocks;
    blocks = cus;
  }
  dim3 grid((unsigned)blocks), block(kNT);
  if (persist) {
    if (K == 128 && V == 128) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 128, false, false, true>), grid, block, 0, s, p);
    else if (K == 64 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 64, false, false, true>), grid, block, 0, s, p);
    else if (K == 128 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 64, false, false, true>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 128, false, false, true>), grid, block, 0, s, p);
  } else if (epi) {
    // progress words from zero (a fill kernel, so that captured graphs clear them too)
    p.prog = reinterpret_cast<unsigned*>(ws + base_need);
    const int frc = launch_fill_zero(p.prog, (int64_t)(norm_prog_bytes(N, HV, V) / 4), s);
    if (frc != GDN_OK) return frc;
    if (K == 128 && V == 128) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 128, false, true>), grid, block, 0, s, p);
    else if (K == 64 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 64, false, true>), grid, block, 0, s, p);
    else if (K == 128 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 64, false, true>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 128, false, true>), grid, block, 0, s, p);
  } else if (chunk_states) {
    if (K == 128 && V == 128) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 128, true>), grid, block, 0, s, p);
    else if (K == 64 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 64, true>), grid, block, 0, s, p);
    else if (K == 128 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 64, true>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 128, true>), grid, block, 0, s, p);
  } else {
    if (K == 128 && V == 128) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 128, false>), grid, block, 0, s, p);
    else if (K == 64 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 64, false>), grid, block, 0, s, p);
    else if (K == 128 && V == 64) hipLaunchKernelGGL((gated_delta_chunk_kernel<128, 64, false>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((gated_delta_chunk_kernel<64, 128, false>), grid, block, 0, s, p);
  }
  const int lrc = gdn_internal_check_launch("gated_delta_chunk_kernel");
  if (lrc != GDN_OK || !norm || epi) return lrc;
  // the norm over the rows just stored, in place (each wave reads its rows before it writes them)
  return gdn_internal_rms_norm_gated(o, ngate, nweight, o, B * T * HV, V, neps, nsplit, s);
}

}  // namespace

extern "C" int gdn_set_range_flag(int device, unsigned* flag) {
  if (device < 0 || device >= kMaxDevices) {
    gdn_internal_set_error("gdn_set_range_flag: device %d out of range", device);
    return GDN_ERR_INVALID;
  }
  unsigned* dptr = nullptr;
  if (flag) {
    hipPointerAttribute_t a{};
    const hipError_t e = hipPointerGetAttributes(&a, flag);
    if (e != hipSuccess || !a.devicePointer ||
        (a.type != hipMemoryTypeHost && !(a.type == hipMemoryTypeDevice && a.device == device))) {
      (void)hipGetLastError();  // a failed query must not surface as the next launch's error
      gdn_internal_set_error("gdn_set_range_flag: the flag must be pinned host memory or memory of device %d", device);
      return GDN_ERR_INVALID;
    }
    dptr = static_cast<unsigned*>(a.devicePointer);
  }
  std::lock_guard<std::mutex> lock(g_flag_mu);
  g_range_flag[device].store(dptr, std::memory_order_release);
  return GDN_OK;
}

extern "C" int gdn_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                             const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                             int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                             int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                             const float* A_log, const float* dt_bias, void* workspace, size_t workspace_bytes,
                             void* stream) {
  return chunk_fwd_impl(q, k, v, g, beta, initial_state, o, final_state, cu_seqlens, B, T, H, HV, K, V, N, qkv_dtype,
                        g_dtype, beta_dtype, scale, flags, A_log, dt_bias, nullptr, workspace, workspace_bytes, stream);
}

extern "C" size_t gdn_chunk_gated_norm_workspace_size(int64_t B, int64_t T, int64_t HV, int64_t N, int64_t V,
                                                      int varlen) {
  const size_t base = gdn_chunk_workspace_size(B, T, HV, N, varlen);
  if (!base || (V != 64 && V != 128)) return 0;
  return base + norm_prog_bytes(N, HV, V);
}

extern "C" int gdn_chunk_fwd_gated_norm(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                        const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                                        int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                                        int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                                        const float* A_log, const float* dt_bias, const void* gate,
                                        const float* norm_weight, float norm_eps, int norm_split, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  if (!gate) {
    gdn_internal_set_error("gdn_chunk_fwd_gated_norm: gate is required");
    return GDN_ERR_INVALID;
  }
  return chunk_fwd_impl(q, k, v, g, beta, initial_state, o, final_state, cu_seqlens, B, T, H, HV, K, V, N, qkv_dtype,
                        g_dtype, beta_dtype, scale, flags, A_log, dt_bias, nullptr, workspace, workspace_bytes, stream,
                        gate, norm_weight, norm_eps, norm_split);
}

extern "C" int gdn_chunk_fwd_train(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                   const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                                   int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                                   int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                                   const float* A_log, const float* dt_bias, void* chunk_states, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (!chunk_states) {
    gdn_internal_set_error("gdn_chunk_fwd_train: chunk_states is required");
    return GDN_ERR_INVALID;
  }
  return chunk_fwd_impl(q, k, v, g, beta, initial_state, o, final_state, cu_seqlens, B, T, H, HV, K, V, N, qkv_dtype,
                        g_dtype, beta_dtype, scale, flags, A_log, dt_bias, chunk_states, workspace, workspace_bytes,
                        stream);
}

// ------------------------------------------------------------------ allocation-free variant
// gdn_chunk_fwd_noalloc runs the same two kernels as gdn_chunk_fwd, with the workspace (the T - I
// rows and the varlen index arrays) in `scratch`, a fixed array in the library's device memory
// instead of a caller buffer. Each device holds its own copy, at its own address, from the load of
// the library until the process ends. In host code `scratch` names a host-side stand-in, not device
// memory: its device address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that address is passed to kernels.
// Nothing in the workspace has to start at zero: the prep kernel writes every T - I row the state
// kernel reads, and the index kernel writes both index arrays. Calls that overlap on one device
// share the array and race.
namespace {

constexpr size_t kScratchBytes = (size_t(64) << 20) + (size_t(64) << 10);  // 64 MiB + 64 KiB
__device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the device that runs `stream` (which must be current).
int scratch_for_stream(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    gdn_internal_set_error("gdn_chunk_fwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return GDN_ERR_HIP;
  }
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) {
      gdn_internal_set_error("gdn_chunk_fwd_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(e));
      return GDN_ERR_HIP;
    }
    if (sdev != dev) {
      gdn_internal_set_error("gdn_chunk_fwd_noalloc: the stream belongs to device %d but device %d is current", sdev,
                             dev);
      return GDN_ERR_INVALID;
    }
  }
  if (dev < 0 || dev >= kMaxDevices) {
    gdn_internal_set_error("gdn_chunk_fwd_noalloc: device %d out of range", dev);
    return GDN_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      gdn_internal_set_error("gdn_chunk_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                             hipGetErrorString(e));
      return GDN_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GDN_OK;
}

}  // namespace

extern "C" size_t gdn_chunk_fwd_noalloc_max_workspace(void) { return kScratchBytes; }

extern "C" int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                     const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                                     int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                                     int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                                     const float* A_log, const float* dt_bias, void* stream) {
  const size_t need = gdn_chunk_workspace_size(B, T, HV, N, cu_seqlens != nullptr);
  if (need > kScratchBytes) {
    gdn_internal_set_error(
        "gdn_chunk_fwd_noalloc: these sizes need %zu bytes of workspace, more than the %zu bytes of the built-in "
        "scratch array (128 bytes per token and value head); use gdn_chunk_fwd with a caller workspace",
        need, kScratchBytes);
    return GDN_ERR_INVALID;
  }
  void* ws = nullptr;
  const int rc = scratch_for_stream(stream, &ws);
  if (rc != GDN_OK) return rc;
  return chunk_fwd_impl(q, k, v, g, beta, initial_state, o, final_state, cu_seqlens, B, T, H, HV, K, V, N, qkv_dtype,
                        g_dtype, beta_dtype, scale, flags, A_log, dt_bias, nullptr, ws, kScratchBytes, stream);
}
