// The T-solve kernel of the chunked prefill (gfx950): for every 64-token chunk and value head,
// T = (I + A)^-1 with A_tj = beta_t exp(gam_t - gam_j) k_t.k_j for j < t (gam = in-chunk cumsum
// of g). This is the UT/WY transform of the chunked gated delta rule
// (oracle/gdn_oracle.py::_chunk_segment restates it; sore/model/gdn_ref.py:17-21 is the recurrence
// it reorganises). T depends only on the chunk's k, g and beta, so every chunk is solved in
// parallel here and the sequential state kernel only reads the result.
//
// One wave per workgroup, sixteen per CU at most (three per SIMD resident), each solving a share
// of one value head's chunks in turn with the next chunk's loads in flight under the current solve.
// The waves never wait for each other, so one wave's serial steps overlap the others' loads and
// MFMAs (gated_delta_chunk_prep_kernel below spells out the steps).

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "gdn_chunk.h"

namespace gdn {

constexpr int kPrepWavesPerCU = 16;  // one-wave T-solve workgroups per CU (three per SIMD fit at once)

// Chunk item -> first token c0 and valid rows len of a value head's chunk; false past the last chunk.
__device__ __forceinline__ bool prep_locate(const ChunkPrepParams& p, int64_t item, int64_t& c0, int& len) {
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
    const uint32_t ncs = (uint32_t)((p.T + kC - 1) / kC), it = (uint32_t)item, q = it / ncs;
    n = q;
    c = it - q * ncs;
    bos = n * p.T;
    eos = bos + p.T;
  }
  c0 = bos + c * kC;
  len = (int)((eos - c0) < kC ? (eos - c0) : kC);
  return true;
}

// The T-solve as one wave per (chunk, value head), with no workgroup barriers between waves: every
// wave of a CU works on its own chunk, so the solve's serial steps (the forward substitutions, the
// chain of block products) of one wave overlap the loads and MFMAs of the others. 10.5 KB of LDS
// and at most 168 VGPRs per wave: three waves per SIMD.
//   load:   the gate bits first (lane = token), then the k rows straight into bf16 MFMA fragments
//           F[rt][s] = K[16rt + i][32s + 8g .. +7] (lane (g, i)), the A operand of row tile rt and
//           equally the B operand of column tile rt; rows past the chunk read as zeros.
//   gates:  in-chunk cumsum (DPP scan) into LDS; the L2 norm of the k rows (when asked) in
//           registers, summed in the order l2norm_row_chunk sums, so the rows are bitwise the ones
//           the state kernel normalises.
//   Gram:   the diagonal tiles K_b K_b^T and, for m < b, K_m K_b^T (40 MFMAs at K = 128). The
//           accumulator of K_m K_b^T holds A[16b + i][16m + 4g + r] once scaled (k.k is symmetric):
//           the row-layout A operand of the block products, so A never passes through LDS.
//   next:   the next chunk's loads, into the registers the Gram has just released.
//   solve:  D_b = (I + A_bb)^-1 by forward substitution in fp32 (lane (column, k) holds rows
//           4q + k), x_m broadcast inside each quad with DPP, the four blocks interleaved; D_b - I
//           to the fp16 staging rows.
//   blocks: T_bc = -D_b sum_{c <= m < b} A_bm T_mc, 16 products of 16x16x16 on
//           v_mfma_f32_16x16x16_f16 (fp16 operands, fp32 sums); each T_mc is an accumulator, which
//           is the B-operand layout, and D_b is read back from the staging rows.
//   store:  T - I as fp16 rows (zeros above the diagonal) in the state kernel's tok_col order.
template <int KD>
__global__ __attribute__((amdgpu_waves_per_eu(3))) __launch_bounds__(kWave) void gated_delta_chunk_prep_kernel(ChunkPrepParams p) {
  constexpr int KS = KD / 32;  // MFMA k-steps over the key dim
  constexpr int KCH = KD / 8;  // 16-byte chunks per k row
  static_assert(KCH == 8 || KCH == 16, "K = 64 or 128");
  // Tb: T - I in natural token order; during the solve its first 4 KB hold the diagonal A blocks,
  // Ad[b][(m * 4 + k) * 4 + q] = A[16b + 4q + k][16b + m].
  __shared__ __align__(16) f16 Tb[kC * kCP];
  __shared__ __align__(16) ChunkGates gs;
  float(*const Ad)[256] = reinterpret_cast<float(*)[256]>(Tb);
  static_assert(sizeof(Tb) >= 4 * 256 * sizeof(float), "Ad fits in Tb");

  const int hv = blockIdx.y, h = hv / (int)(p.HV / p.H);
  const uint32_t row_b = (uint32_t)(p.H * KD * 2);
  // the gate bits (lane = token) and the k fragments of a chunk; rows past its end read as zeros.
  // Lane ids come through opaque_int wherever they are used in the loop, so the address arithmetic
  // is recomputed per chunk instead of being hoisted into registers held across the loop.
  uint32_t graw = 0, braw = 0;
  bf16x8 F[4][KS];
  auto issue_loads = [&](int64_t c0, int len, int ln) {
    graw = braw = 0;
    if (ln < len) {
      const int64_t gi = (c0 + ln) * p.HV + hv;
      graw = load_raw32(p.g, p.dg, gi);
      braw = load_raw32(p.beta, p.db, gi);
    }
    const auto rk = make_rsrc(static_cast<const bf16*>(p.k) + (c0 * p.H + h) * KD, (uint32_t)len * row_b);
    const int lg = ln >> 4, lr = ln & 15;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int s = 0; s < KS; ++s) F[rt][s] = buf_load16(rk, (uint32_t)(16 * rt + lr) * row_b + (uint32_t)(32 * s + 8 * lg) * 2);
  };
  // The wave solves the chunks blockIdx.x, blockIdx.x + gridDim.x, ... of its value head. The next
  // chunk's loads go out once the current one's k fragments are in the Gram MFMAs (gates first:
  // the scan then waits only for them), so their latency hides under the solve.
  int64_t item = blockIdx.x, c0 = 0;
  int len = 0;
  bool valid = prep_locate(p, item, c0, len);
  if (valid) issue_loads(c0, len, (int)threadIdx.x);
  while (valid) {
  const int lane = opaque_int((int)threadIdx.x), g4 = lane >> 4, li = lane & 15;
  chunk_gates_from_raw(gs, graw, braw, p.dg, p.db, len, p.flags, p.A_log ? p.A_log[hv] : 0.f,
                       p.dt_bias ? p.dt_bias[hv] : 0.f, lane);

  if (p.flags & GDN_FLAG_QK_L2NORM) {
    // row 16rt + i spans chunks 4s + g of its KCH: the pair sums over g (lanes 16 and 32 apart) then
    // over s reproduce group_sum<KCH>'s tree (chunk ^ 1, ^ 2, ^ 4, ^ 8)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      float v[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)F[rt][s][e] * (float)F[rt][s][e];
        v[s] = ss;
      }
#pragma unroll
      for (int s = 0; s < KS; ++s) v[s] += __shfl_xor(v[s], 16, kWave);
#pragma unroll
      for (int s = 0; s < KS; ++s) v[s] += __shfl_xor(v[s], 32, kWave);
      float tot;
      if constexpr (KS == 4) tot = (v[0] + v[1]) + (v[2] + v[3]);
      else tot = v[0] + v[1];
      const float inv = __builtin_amdgcn_rsqf(fmaxf(tot, 1e-24f));
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) F[rt][s][e] = static_cast<bf16>((float)F[rt][s][e] * inv);
    }
  }

  // ---------------------------------------------------------------- Gram tiles
  // Gd[b]: K_b K_b^T (symmetric): element (row 4g + r, column i) read as k_{16b+i}.k_{16b+4g+r}.
  // Go[o(b, m)], m < b: K_m K_b^T, element (4g + r, i) = k_{16b+i}.k_{16m+4g+r}.
  constexpr int kO = 6;
  auto oidx = [](int b, int m) { return b * (b - 1) / 2 + m; };
  f32x4 Gd[4], Go[kO];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    Gd[b] = f32x4{};
#pragma unroll
    for (int s = 0; s < KS; ++s) Gd[b] = mma(F[b][s], F[b][s], Gd[b]);
  }
#pragma unroll
  for (int b = 1; b < 4; ++b)
#pragma unroll
    for (int m = 0; m < b; ++m) {
      f32x4 acc{};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = mma(F[m][s], F[b][s], acc);
      Go[oidx(b, m)] = acc;
    }
  const int64_t next = item + gridDim.x;
  int64_t nc0 = 0;
  int nlen = 0;
  const bool nvalid = prep_locate(p, next, nc0, nlen);
  if (nvalid) issue_loads(nc0, nlen, opaque_int((int)threadIdx.x));
  __syncthreads();  // gs written by the scan above

  // ---------------------------------------------------------------- A = beta_t exp(gam_t - gam_j) k_t.k_j, j < t
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float gt = gs.gam[16 * b + li], bt = gs.bet[16 * b + li];
    // diagonal block: A[16b + i][16b + 4g + r] for 4g + r < i, to Ad in the solve's layout
    const float4 gj = ld4f(&gs.gam[16 * b + 4 * g4]);
    const float gjv[4] = {gj.x, gj.y, gj.z, gj.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float av = (4 * g4 + r < li) ? bt * __expf(gt - gjv[r]) * Gd[b][r] : 0.f;
      Ad[b][((4 * g4 + r) * 4 + (li & 3)) * 4 + (li >> 2)] = av;
    }
    // off-diagonal blocks in row layout: lane (g, i) holds A[16b + i][16m + 4g + r]
#pragma unroll
    for (int m = 0; m < b; ++m) {
      const float4 gm = ld4f(&gs.gam[16 * m + 4 * g4]);
      const float gmv[4] = {gm.x, gm.y, gm.z, gm.w};
      f32x4& a = Go[oidx(b, m)];
#pragma unroll
      for (int r = 0; r < 4; ++r) a[r] = bt * __expf(gt - gmv[r]) * a[r];
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- diagonal inverses
  // Lane (col, k) = (lane / 4, lane % 4) holds x[b][q] = D_b[4q + k][col]; step m broadcasts x_m
  // inside each quad and reads the lane's four A entries of column m with one 16-byte LDS read. The
  // four blocks' substitutions are interleaved step by step (independent chains).
  const int col = lane >> 2, kq = lane & 3;
  float x[4][4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int q = 0; q < 4; ++q) x[b][q] = (4 * q + kq == col) ? 1.f : 0.f;
  // the A entries of step m + 1 are read during step m (two register sets); the scheduler may not
  // hoist reads further (sched_barrier), which would hold up to 240 registers of A entries
  float4 a4n[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) a4n[b] = ld4f(&Ad[b][kq * 4]);
#pragma unroll
  for (int m = 0; m < 15; ++m) {
    float4 a4[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) a4[b] = a4n[b];
    if (m + 1 < 15) {
#pragma unroll
      for (int b = 0; b < 4; ++b) a4n[b] = ld4f(&Ad[b][((m + 1) * 4 + kq) * 4]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float xm = quad_bcast(x[b][m >> 2], m & 3);
      // rows 4q + k <= m have A[4q + k][m] = 0: the groups q with 4q + 3 <= m are left alone
      if (4 * 0 + 3 > m) x[b][0] -= a4[b].x * xm;
      if (4 * 1 + 3 > m) x[b][1] -= a4[b].y * xm;
      if (4 * 2 + 3 > m) x[b][2] -= a4[b].z * xm;
      x[b][3] -= a4[b].w * xm;
    }
  }
  __syncthreads();  // Ad is dead: Tb takes its space
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rr = 4 * q + kq;
      Tb[(16 * b + rr) * kCP + 16 * b + col] = static_cast<f16>(rr == col ? 0.f : x[b][q]);
    }
  __syncthreads();

  // ---------------------------------------------------------------- off-diagonal blocks of T
  // T_bc = -D_b sum_{c <= m < b} A_bm T_mc with fp16 operands and fp32 accumulation
  // (v_mfma_f32_16x16x16_f16: A lane (g, i) holds row i, k = 4g..4g+3; B and the accumulator hold
  // column i, rows 4g..4g+3). T is stored in fp16, and rounding the products' operands to fp16
  // as well keeps T within 1.4e-4 of its fp64 value relative to max|T| (6e-5 from the storage
  // rounding alone) over config-1 chunk statistics. D_b comes back from its fp16 rows in Tb (the
  // diagonal, stored as 0, read as 1): as an A operand by row, as a B operand by transposed read.
  auto unit_diag = [&](f16x4 v) {  // adds the identity: element r sits on the diagonal when 4g + r == i
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * g4 + r == li) v[r] = static_cast<f16>(1.f);
    return v;
  };
  auto d_row = [&](int b) { return unit_diag(*reinterpret_cast<const f16x4*>(&Tb[(16 * b + li) * kCP + 16 * b + 4 * g4])); };
  auto d_acc = [&](int b) {
    const bf16x4 v = ld4_tr(reinterpret_cast<const bf16*>(Tb), kCP, 16 * b, 16 * b, lane);
    return unit_diag(__builtin_bit_cast(f16x4, v));
  };
  auto to_h4 = [](const f32x4& t) { return to_f16x4(t[0], t[1], t[2], t[3]); };
  auto mma16h = [](f16x4 a, f16x4 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); };
  f16x4 Ah[kO], Th[kO];  // A_bm in row layout; T_bc, b > c, in accumulator layout (fp16)
#pragma unroll
  for (int o = 0; o < kO; ++o) Ah[o] = to_h4(Go[o]);
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const f16x4 dc = d_acc(c);
#pragma unroll
    for (int b = c + 1; b < 4; ++b) {
      f32x4 w{};
#pragma unroll
      for (int m = c; m < b; ++m) w = mma16h(Ah[oidx(b, m)], m == c ? dc : Th[oidx(m, c)], w);
      const f32x4 t = mma16h(d_row(b), to_h4(w), f32x4{});
      Th[oidx(b, c)] = to_f16x4(-t[0], -t[1], -t[2], -t[3]);
    }
  }
#pragma unroll
  for (int c = 0; c < 3; ++c)
#pragma unroll
    for (int b = c + 1; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) Tb[(16 * b + 4 * g4 + r) * kCP + 16 * c + li] = Th[oidx(b, c)][r];
  __syncthreads();

  // ---------------------------------------------------------------- store rows t < len
  // The 16 bytes at columns 8p..8p+7, p = 4u + g, hold the tokens 32u + 4g + 0..3 and
  // 32u + 16 + 4g + 0..3 (tok_col); a half whose 16x16 block lies above the diagonal is zero.
  f16* const tw = p.tw + (c0 * p.HV + hv) * kC;
#pragma unroll
  for (int u = 0; u < kC * 8 / kWave; ++u) {
    const int e = lane + u * kWave, row = e >> 3, p8 = e & 7;
    if (row < len) {
      const int j0 = 32 * (p8 >> 2) + 4 * (p8 & 3), j1 = j0 + 16;
      const f16x4 a = (j0 >> 4) > (row >> 4) ? f16x4{} : *reinterpret_cast<const f16x4*>(&Tb[row * kCP + j0]);
      const f16x4 b = (j1 >> 4) > (row >> 4) ? f16x4{} : *reinterpret_cast<const f16x4*>(&Tb[row * kCP + j1]);
      *reinterpret_cast<f16x8*>(tw + (int64_t)row * p.HV * kC + p8 * 8) = f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
  }
  __syncthreads();  // Tb is read before the next chunk's A blocks take its space
  item = next;
  c0 = nc0;
  len = nlen;
  valid = nvalid;
  }
}

// One block of nt = 64..1024 threads (a multiple of 64, sized to N by the launcher: one wave for up
// to 64 sequences, whose barriers are then nearly free), with cu_seqlens:
//   chunk_first[0] = 0, chunk_first[n + 1] = chunk_first[n] + ceil(len_n / 64) (a running block-wide
//   scan over tiles of nt sequences): the prep kernel's chunk -> sequence map;
//   order[k] = the sequence of rank k by length, longest first (ties by index), for N <= kOrderMax
//   (a bitonic sort in LDS; identity above that): the state kernel starts the longest recurrences
//   first, so a grid larger than the machine finishes near the longest sequence's own time.
__global__ __launch_bounds__(1024) void gated_delta_chunk_index_kernel(const void* cu, int cu_i32, int64_t N,
                                                                        int* chunk_first, int* order) {
  __shared__ int wsum[16];
  __shared__ int carry;
  __shared__ unsigned long long keys[kOrderMax];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, nt = (int)blockDim.x;
  if (t == 0) {
    carry = 0;
    chunk_first[0] = 0;
  }
  __syncthreads();
  for (int64_t base = 0; base < N; base += nt) {
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
    if (t == nt - 1) carry = before + incl;
    __syncthreads();
  }
  if (N > kOrderMax) {
    for (int64_t n = t; n < N; n += nt) order[n] = (int)n;
    return;
  }
  // key = (chunks descending, index ascending); padding sorts last
  int m = 1;
  while (m < N) m <<= 1;
  for (int n = t; n < m; n += nt) {
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
      for (int n = t; n < m; n += nt) {
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
  for (int n = t; n < N; n += nt) order[n] = (int)(keys[n] & 0xffffffffu);
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

int device_compute_units(hipStream_t s) { return device_cus(s); }

// Threads of the index kernel's block for N sequences: N rounded up to a wave, at most 1024.
static unsigned index_threads(int64_t N) { return (unsigned)std::min<int64_t>(1024, std::max<int64_t>(1, (N + 63) / 64) * 64); }

int launch_chunk_index(const void* cu, int cu_i32, int64_t N, int* chunk_first, int* order, hipStream_t s) {
  hipLaunchKernelGGL(gated_delta_chunk_index_kernel, dim3(1), dim3(index_threads(N)), 0, s, cu, cu_i32, N, chunk_first,
                     order);
  return gdn_internal_check_launch("gated_delta_chunk_index_kernel");
}

int launch_chunk_prep(const ChunkPrepParams& prm, int64_t B, int64_t K, hipStream_t s) {
  ChunkPrepParams p = prm;
  if (p.cu) {
    hipLaunchKernelGGL(gated_delta_chunk_index_kernel, dim3(1), dim3(index_threads(p.N)), 0, s, p.cu, p.cu_i32, p.N,
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
  // One wave per workgroup, about kPrepWavesPerCU per CU, each walking an equal share of its value
  // head's chunks with stride gridDim.x (waves past the last chunk return at once).
  static const int64_t wpc = [] {
    const char* e = getenv("SORERNN_TSOLVE_WPC");
    return (int64_t)(e ? std::max(1, atoi(e)) : kPrepWavesPerCU);
  }();
  const int64_t slots = wpc * (int64_t)device_cus(s);
  const int64_t gx0 = std::max<int64_t>(1, std::min<int64_t>(p.items, (slots + p.HV - 1) / p.HV));
  const int64_t per = std::max<int64_t>(1, (p.items + gx0 - 1) / gx0);
  const int64_t gx = std::max<int64_t>(1, (p.items + per - 1) / per);
  dim3 grid((unsigned)gx, (unsigned)p.HV), block(kWave);
  if (K == 128) hipLaunchKernelGGL(gated_delta_chunk_prep_kernel<128>, grid, block, 0, s, p);
  else hipLaunchKernelGGL(gated_delta_chunk_prep_kernel<64>, grid, block, 0, s, p);
  return gdn_internal_check_launch("gated_delta_chunk_prep_kernel");
}

}  // namespace gdn
