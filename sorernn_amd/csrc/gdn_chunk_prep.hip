// The T-solve kernel of the chunked prefill (gfx950): for every 64-token chunk and value head,
// T = (I + A)^-1 with A_tj = beta_t exp(gam_t - gam_j) k_t.k_j for j < t (gam = in-chunk cumsum
// of g). This is the UT/WY transform of the chunked gated delta rule
// (oracle/gdn_oracle.py::_chunk_segment restates it; sore/model/gdn_ref.py:17-21 is the recurrence
// it reorganises). T depends only on the chunk's k, g and beta, so every chunk is solved in
// parallel here and the sequential state kernel only reads the result.
//
// Workgroups of 4 waves, about four per CU, each solving a share of one value head's chunks in turn
// (the next chunk's loads in flight under the current solve):
//   load:   k rows (L2-normalised when asked, rounded to bf16 as the state kernel sees them) -> LDS;
//           g/beta -> gate terms (wave 0, DPP scan).
//   Gram:   wave r computes the 16x16 k.k tiles (r, cb >= r) with bf16 MFMA (exact products, fp32
//           sums), scales them into A, and solves its diagonal block T_rr = (I + A_rr)^-1 by
//           forward substitution on 64 lanes (fp32).
//   merge:  T_{2q+1,2q} = -T_{2q+1,2q+1} A_{2q+1,2q} T_{2q,2q} (16 -> 32), then the 32 -> 64
//           block, with fp32 MFMA products (v_mfma_f32_16x16x4_f32).
//   store:  rows of T - I (fp16, zeros above the diagonal) to the workspace, one 128-byte row per
//           token with the columns in the state kernel's contraction order (tok_col): the A
//           operand of Delta = X + (T - I) X there.

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

constexpr int kPrepNT = 256;

template <int KD>
__global__ __launch_bounds__(kPrepNT, 4) void gated_delta_chunk_prep_kernel(ChunkPrepParams p) {
  constexpr int KP = KD + 8;   // bf16 pitch of the k tile
  constexpr int KS = KD / 32;  // MFMA k-steps over the key dim
  constexpr int KCH = KD / 8;  // 16-byte chunks per k row
  constexpr int KPT = kC * KCH / kPrepNT;

  // The k tile is dead once the Gram MFMAs have read it, so the solve's buffers reuse its space
  // (about 34 KB per workgroup in all: four workgroups fit a CU's LDS):
  //   Ad  diagonal A blocks: Ad[b][(4m + k) * 4 + q] = A[16b+4q+k][16b+m]
  //   Ao  A rows 16..63 x cols 0..47 (the off-diagonal lower blocks)
  //   Tf  T[0:32][0:32] and T[32:64][32:64] in fp32
  //   Tb  T - I in fp16 [t][j] (blocks above the diagonal are never written: the store zero-fills them)
  constexpr int kAdB = 4 * 256 * 4, kAoB = 48 * kAoP * 4, kTfB = 2 * 32 * kTfP * 4, kTbB = kC * kCP * 2;
  constexpr int kSolveB = kAdB + kAoB + kTfB + kTbB, kKcB = kC * KP * 2;
  __shared__ __align__(16) char smem[kSolveB > kKcB ? kSolveB : kKcB];
  __shared__ __align__(16) ChunkGates gs;
  bf16* const Kc = reinterpret_cast<bf16*>(smem);
  float(*const Ad)[256] = reinterpret_cast<float(*)[256]>(smem);
  float* const Ao = reinterpret_cast<float*>(smem + kAdB);
  float(*const Tf)[32 * kTfP] = reinterpret_cast<float(*)[32 * kTfP]>(smem + kAdB + kAoB);
  f16* const Tb = reinterpret_cast<f16*>(smem + kAdB + kAoB + kTfB);

  const int tid = threadIdx.x, w = tid >> 6;
  const int hv = blockIdx.y;
  const int h = hv / (int)(p.HV / p.H);
  const bf16* __restrict__ kg = static_cast<const bf16*>(p.k);

  // chunk item -> first token c0 and valid rows len; false past the last chunk
  auto locate = [&](int64_t item, int64_t& c0, int& len) -> bool {
    int64_t n, c, bos, eos;
    if (p.cu) {
      // largest n with chunk_first[n] <= item (skips empty sequences)
      if (item >= p.chunk_first[p.N]) return false;
      int64_t lo = 0, hi = p.N - 1;
      while (lo < hi) {
        const int64_t mid = (lo + hi + 1) / 2;
        if (p.chunk_first[mid] <= item) lo = mid;
        else hi = mid - 1;
      }
      n = lo;
      c = item - p.chunk_first[n];
      bos = load_index(p.cu, p.cu_i32, n);
      eos = load_index(p.cu, p.cu_i32, n + 1);
    } else {
      if (item >= p.items) return false;
      // 32-bit division (items < 2^31, checked at launch): the 64-bit one expands to a few hundred
      // instructions, paid for every chunk a workgroup walks
      const uint32_t ncs = (uint32_t)((p.T + kC - 1) / kC), it = (uint32_t)item, q = it / ncs;
      n = q;
      c = it - q * ncs;
      bos = n * p.T;
      eos = bos + p.T;
    }
    c0 = bos + c * kC;
    len = (int)((eos - c0) < kC ? (eos - c0) : kC);
    return true;
  };
  // the k rows and raw gate bits of a chunk, into registers
  bf16x8 kv[KPT];
  uint32_t graw = 0, braw = 0;
  auto issue_loads = [&](int64_t c0, int len) {
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int e = tid + u * kPrepNT, row = e / KCH, c8 = e % KCH;
      kv[u] = bf16x8{};
      if (row < len) kv[u] = *reinterpret_cast<const bf16x8*>(kg + ((c0 + row) * p.H + h) * KD + c8 * 8);
    }
    graw = braw = 0;
    if (w == 0 && tid < len) {
      const int64_t gi = (c0 + tid) * p.HV + hv;
      graw = load_raw32(p.g, p.dg, gi);
      braw = load_raw32(p.beta, p.db, gi);
    }
  };

  // The workgroup solves the chunks blockIdx.x, blockIdx.x + gridDim.x, ... of its value head; the
  // loads of the next chunk are issued once the current one's k rows are in the Gram MFMAs, so
  // their latency hides under the solve.
  int64_t item = blockIdx.x, c0 = 0;
  int len = 0;
  bool valid = locate(item, c0, len);
  if (valid) issue_loads(c0, len);
  while (valid) {
    // lane ids through an opaque copy per chunk: the solve's address arithmetic is recomputed in each
    // pass rather than hoisted out of the loop into registers held across it
    const int t = opaque_int(tid), lane = t & 63, g4 = lane >> 4, li = lane & 15;
    // ------------------------------------------------------------------ stage
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int e = t + u * kPrepNT, row = e / KCH, c8 = e % KCH;
      const bf16x8 x = (p.flags & GDN_FLAG_QK_L2NORM) ? l2norm_row_chunk<KCH>(kv[u]) : kv[u];
      *reinterpret_cast<bf16x8*>(&Kc[row * KP + c8 * 8]) = x;
    }
    if (w == 0)
      chunk_gates_from_raw(gs, graw, braw, p.dg, p.db, len, p.flags, p.A_log ? p.A_log[hv] : 0.f,
                           p.dt_bias ? p.dt_bias[hv] : 0.f, lane);
    __syncthreads();

    // ------------------------------------------------------------------ Gram tiles, A, diagonal solves
    // Wave r: row tile r of A (a template constant: one code copy per wave). The k.k tiles stay in
    // registers across the barrier that retires the k tile.
    f32x4 dacc{}, oacc[3] = {};
    auto gram_mfma = [&](auto rc) {
      constexpr int rk = decltype(rc)::value;
      bf16x8 fk[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) fk[s] = ld8(Kc + (16 * rk + li) * KP + 32 * s + 8 * g4);
#pragma unroll
      for (int s = 0; s < KS; ++s) dacc = mma(fk[s], fk[s], dacc);
#pragma unroll
      for (int cb = rk + 1; cb < 4; ++cb) {
        bf16x8 fo[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) fo[s] = ld8(Kc + (16 * cb + li) * KP + 32 * s + 8 * g4);
#pragma unroll
        for (int s = 0; s < KS; ++s) oacc[cb - 1] = mma(fk[s], fo[s], oacc[cb - 1]);
      }
    };
    auto gram_post = [&](auto rc) {
      constexpr int rk = decltype(rc)::value;
      // k.k is symmetric: dacc[i] = k_t.k_j with t = 16rk + li, j = 16rk + 4g + i; A[t][j] for j < t
      const float gt = gs.gam[16 * rk + li], bt = gs.bet[16 * rk + li];
      const float4 gj = ld4f(&gs.gam[16 * rk + 4 * g4]);
      const float gjv[4] = {gj.x, gj.y, gj.z, gj.w};
      float av[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) av[ii] = (4 * g4 + ii < li) ? bt * __expf(gt - gjv[ii]) * dacc[ii] : 0.f;
      // A_rr, stored for the solve as ad[m][k][q] = A[4q + k][m] (private to this wave)
      float* ad = Ad[rk];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) ad[((4 * g4 + ii) * 4 + (li & 3)) * 4 + (li >> 2)] = av[ii];
      // off-diagonal A blocks: element (j = 16rk + 4g + i, t = 16cb + li) -> Ao[t - 16][j]
#pragma unroll
      for (int cb = rk + 1; cb < 4; ++cb) {
        const int tt = 16 * cb + li, j0 = 16 * rk + 4 * g4;
        const float gtt = gs.gam[tt], btt = gs.bet[tt];
        float val[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) val[ii] = btt * __expf(gtt - gjv[ii]) * oacc[cb - 1][ii];
        *reinterpret_cast<float4*>(&Ao[(tt - 16) * kAoP + j0]) = make_float4(val[0], val[1], val[2], val[3]);
      }
      // Forward substitution on 64 lanes: lane (col = lane/4, k = lane%4) holds rows 4q+k of column
      // col of T_rr; x_m is broadcast inside each quad with DPP, and step m reads the lane's four A
      // entries of column m with one 16-byte LDS read. A is strictly lower, so no row mask is needed.
      const int col = lane >> 2, kq = lane & 3;
      float4 a4m[15];
#pragma unroll
      for (int m = 0; m < 15; ++m) a4m[m] = ld4f(ad + (m * 4 + kq) * 4);
      float x[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) x[q] = (4 * q + kq == col) ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < 15; ++m) {
        const float xm = quad_bcast(x[m >> 2], m & 3);
        x[0] -= a4m[m].x * xm;
        x[1] -= a4m[m].y * xm;
        x[2] -= a4m[m].z * xm;
        x[3] -= a4m[m].w * xm;
      }
      float* tf = &Tf[rk >> 1][(16 * (rk & 1)) * kTfP + 16 * (rk & 1) + col];
      f16* tb = &Tb[(16 * rk) * kCP + 16 * rk + col];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rr = 4 * q + kq;
        tf[rr * kTfP] = x[q];
        tb[rr * kCP] = static_cast<f16>(rr == col ? 0.f : x[q]);
      }
    };
    switch (w) {
      case 0: gram_mfma(std::integral_constant<int, 0>{}); break;
      case 1: gram_mfma(std::integral_constant<int, 1>{}); break;
      case 2: gram_mfma(std::integral_constant<int, 2>{}); break;
      default: gram_mfma(std::integral_constant<int, 3>{}); break;
    }
    // the next chunk's loads (kv and the raw gates have been consumed by the stage above)
    const int64_t next = item + gridDim.x;
    int64_t nc0 = 0;
    int nlen = 0;
    const bool nvalid = locate(next, nc0, nlen);
    if (nvalid) issue_loads(nc0, nlen);
    __syncthreads();  // the k tile is dead from here on
    switch (w) {
      case 0: gram_post(std::integral_constant<int, 0>{}); break;
      case 1: gram_post(std::integral_constant<int, 1>{}); break;
      case 2: gram_post(std::integral_constant<int, 2>{}); break;
      default: gram_post(std::integral_constant<int, 3>{}); break;
    }
    __syncthreads();

    // ------------------------------------------------------------------ 16 -> 32 merges (waves 2, 3)
    // T_{2q+1,2q} = -T_{2q+1,2q+1} (A_{2q+1,2q} T_{2q,2q}). W = A T_{2q,2q} lands in accumulator layout,
    // which is the B-operand layout of the product step (mma16f), so the second product takes W from registers.
    if (w >= 2) {
      const int q = w - 2;
      const float* tq = Tf[q];
      f32x4 acc{};
      {
        float a[4], b[4];
        const float* ar = &Ao[(16 * (2 * q + 1) + li - 16) * kAoP + 32 * q + 4 * g4];
        a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
#pragma unroll
        for (int m = 0; m < 4; ++m) b[m] = tq[(4 * g4 + m) * kTfP + li];
        acc = mma16f(a, b, acc);
      }
      f32x4 acc2{};
      {
        float a[4];
        const float b[4] = {acc[0], acc[1], acc[2], acc[3]};
        const float* ar = &tq[(16 + li) * kTfP + 16 + 4 * g4];
        a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
        acc2 = mma16f(a, b, acc2);
      }
      float* tw = &Tf[q][16 * kTfP];
      f16* tbw = &Tb[(32 * q + 16) * kCP + 32 * q];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        tw[(4 * g4 + ii) * kTfP + li] = -acc2[ii];
        tbw[(4 * g4 + ii) * kCP + li] = static_cast<f16>(-acc2[ii]);
      }
    }
    __syncthreads();

    // ------------------------------------------------------------------ 32 -> 64 merge (waves 2, 3)
    // T[32:64][0:32] = -T[32:64][32:64] (A[32:64][0:32] T[0:32][0:32]), column block ct = w - 2.
    if (w >= 2) {
      const int ct = w - 2;
      f32x4 wacc[2];  // W' tiles (rt, ct), kept in registers as the B operand of the second product
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        wacc[rt] = f32x4{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if (ks < ct) continue;  // T[k][c] vanishes for k < c
          float a[4], b[4];
          const float* ar = &Ao[(16 + 16 * rt + li) * kAoP + 16 * ks + 4 * g4];
          a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
#pragma unroll
          for (int m = 0; m < 4; ++m) b[m] = Tf[0][(16 * ks + 4 * g4 + m) * kTfP + 16 * ct + li];
          wacc[rt] = mma16f(a, b, wacc[rt]);
        }
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        f32x4 acc{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if (ks > rt) continue;  // T[32+r][32+k] vanishes for k > r
          float a[4];
          const float b[4] = {wacc[ks][0], wacc[ks][1], wacc[ks][2], wacc[ks][3]};
          const float* ar = &Tf[1][(16 * rt + li) * kTfP + 16 * ks + 4 * g4];
          a[0] = ar[0]; a[1] = ar[1]; a[2] = ar[2]; a[3] = ar[3];
          acc = mma16f(a, b, acc);
        }
        f16* tbw = &Tb[(32 + 16 * rt) * kCP + 16 * ct];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) tbw[(4 * g4 + ii) * kCP + li] = static_cast<f16>(-acc[ii]);
      }
    }
    __syncthreads();

    // ------------------------------------------------------------------ store rows t < len
    // Columns in the state kernel's contraction order (tok_col): the 16 bytes at columns 8p..8p+7,
    // p = 4u + g, hold the tokens 32u + 4g + 0..3 and 32u + 16 + 4g + 0..3. A piece whose 16x16 block
    // lies above the diagonal is zero.
#pragma unroll
    for (int u = 0; u < kC * 8 / kPrepNT; ++u) {
      const int e = t + u * kPrepNT, row = e >> 3, p8 = e & 7;
      if (row < len) {
        const int j0 = 32 * (p8 >> 2) + 4 * (p8 & 3), j1 = j0 + 16;
        const f16x4 a = (j0 >> 4) > (row >> 4) ? f16x4{} : *reinterpret_cast<const f16x4*>(&Tb[row * kCP + j0]);
        const f16x4 b = (j1 >> 4) > (row >> 4) ? f16x4{} : *reinterpret_cast<const f16x4*>(&Tb[row * kCP + j1]);
        *reinterpret_cast<f16x8*>(p.tw + ((c0 + row) * p.HV + hv) * kC + p8 * 8) =
            f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
      }
    }
    __syncthreads();  // Tb is read before the next chunk's k rows take its space
    item = next;
    c0 = nc0;
    len = nlen;
    valid = nvalid;
  }
}

// One block, with cu_seqlens:
//   chunk_first[0] = 0, chunk_first[n + 1] = chunk_first[n] + ceil(len_n / 64) (a running block-wide
//   scan over tiles of 1024 sequences): the prep kernel's chunk -> sequence map;
//   order[k] = the sequence of rank k by length, longest first (ties by index), for N <= kOrderMax
//   (a bitonic sort in LDS; identity above that): the state kernel starts the longest recurrences
//   first, so a grid larger than the machine finishes near the longest sequence's own time.
constexpr int kOrderMax = 2048;
__global__ __launch_bounds__(1024) void gated_delta_chunk_index_kernel(const void* cu, int cu_i32, int64_t N,
                                                                        int* chunk_first, int* order) {
  __shared__ int wsum[16];
  __shared__ int carry;
  __shared__ unsigned long long keys[kOrderMax];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (t == 0) {
    carry = 0;
    chunk_first[0] = 0;
  }
  __syncthreads();
  for (int64_t base = 0; base < N; base += 1024) {
    const int64_t n = base + t;
    int v = 0;
    if (n < N) v = (int)((load_index(cu, cu_i32, n + 1) - load_index(cu, cu_i32, n) + kC - 1) / kC);
    int incl = v;  // inclusive scan inside the wave
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) wsum[w] = incl;
    __syncthreads();
    int before = carry;
    for (int j = 0; j < w; ++j) before += wsum[j];
    if (n < N) chunk_first[n + 1] = before + incl;
    __syncthreads();
    if (t == 1023) carry = before + incl;
    __syncthreads();
  }
  if (N > kOrderMax) {
    for (int64_t n = t; n < N; n += 1024) order[n] = (int)n;
    return;
  }
  // key = (chunks descending, index ascending); padding sorts last
  int m = 1;
  while (m < N) m <<= 1;
  for (int n = t; n < m; n += 1024) {
    unsigned long long key = ~0ull;
    if (n < N) {
      const unsigned nch = (unsigned)((load_index(cu, cu_i32, n + 1) - load_index(cu, cu_i32, n) + kC - 1) / kC);
      key = ((unsigned long long)(0xffffffffu - nch) << 32) | (unsigned)n;
    }
    keys[n] = key;
  }
  __syncthreads();
  for (int size = 2; size <= m; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int n = t; n < m; n += 1024) {
        const int partner = n ^ stride;
        if (partner > n) {
          const bool up = (n & size) == 0;
          const unsigned long long a = keys[n], b = keys[partner];
          if ((a > b) == up) {
            keys[n] = b;
            keys[partner] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int n = t; n < N; n += 1024) order[n] = (int)(keys[n] & 0xffffffffu);
}

namespace {

constexpr int kMaxCuCache = 64;
std::atomic<int> g_cus[kMaxCuCache] = {};

// Compute units of the device that runs `s` (looked up once per device; 256 on MI355X).
int device_cus(hipStream_t s) {
  int dev = 0;
  if ((s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev)) != hipSuccess || dev < 0 || dev >= kMaxCuCache) return 256;
  int v = g_cus[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    g_cus[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace

int launch_chunk_index(const void* cu, int cu_i32, int64_t N, int* chunk_first, int* order, hipStream_t s) {
  hipLaunchKernelGGL(gated_delta_chunk_index_kernel, dim3(1), dim3(1024), 0, s, cu, cu_i32, N, chunk_first, order);
  return gdn_internal_check_launch("gated_delta_chunk_index_kernel");
}

int launch_chunk_prep(const ChunkPrepParams& prm, int64_t B, int64_t K, hipStream_t s) {
  ChunkPrepParams p = prm;
  if (p.cu) {
    hipLaunchKernelGGL(gated_delta_chunk_index_kernel, dim3(1), dim3(1024), 0, s, p.cu, p.cu_i32, p.N,
                       const_cast<int*>(p.chunk_first), const_cast<int*>(p.order));
    p.items = (p.T + kC - 1) / kC + p.N;  // upper bound on the number of chunks
  } else {
    p.items = B * ((p.T + kC - 1) / kC);
  }
  if (p.items > 0x7fffffff || p.HV > 65535) {
    gdn_internal_set_error("gdn_chunk_fwd: %lld chunks x %lld heads exceed the grid limits", (long long)p.items,
                           (long long)p.HV);
    return GDN_ERR_UNSUPPORTED;
  }
  // About four workgroups per CU (the LDS holds four), each walking an equal share of its value
  // head's chunks with stride gridDim.x.
  const int64_t slots = 4 * (int64_t)device_cus(s);
  const int64_t gx0 = std::max<int64_t>(1, std::min<int64_t>(p.items, (slots + p.HV - 1) / p.HV));
  const int64_t per = std::max<int64_t>(1, (p.items + gx0 - 1) / gx0);
  const int64_t gx = std::max<int64_t>(1, (p.items + per - 1) / per);
  dim3 grid((unsigned)gx, (unsigned)p.HV), block(kPrepNT);
  if (K == 128) hipLaunchKernelGGL(gated_delta_chunk_prep_kernel<128>, grid, block, 0, s, p);
  else hipLaunchKernelGGL(gated_delta_chunk_prep_kernel<64>, grid, block, 0, s, p);
  return gdn_internal_check_launch("gated_delta_chunk_prep_kernel");
}

}  // namespace gdn
