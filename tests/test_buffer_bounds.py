"""CPU model of the byte ranges the chunked-prefill kernels touch in HBM.

The chunk kernels (``gdn_chunk.hip``, ``gdn_chunk_prep.hip``, ``gdn_chunk_bwd.hip``) load most
tiles through buffer resources and rely on the hardware range check for rows past a chunk's end.
That check only guarantees that nothing beyond ``base + num_records`` is touched; it does not
stop a load whose resource itself, or whose width, extends past the tensor. This module restates,
for every resource and plain global access of those kernels, the resource base, its size, the
per-lane offsets and the access width, and checks at the BASELINE shapes (configs 1, 3, 4), ragged
and GVA cases, with fp32 and bf16 gates, that every access which can execute lies inside its
tensor.

The check is deliberately permissive about the hardware: an access counts as executed whenever
its first byte is inside the resource (the weakest range-check convention), and then every byte of
it must be inside the tensor.

``test_checker_flags_the_old_gate_loads`` keeps the gate-load scheme the state kernel used before
(a 32-bit load at every 16-bit gate, through a resource of len * HV * 2 bytes from the head's
first element) as a negative control: it read 2 bytes past the end of a bf16 gate tensor, and the
checker must flag it. ``test_model_covers_every_buffer_resource`` ties the model to the sources by
counting the buffer resources each kernel file creates.
"""
from __future__ import annotations

import os
import re
from dataclasses import dataclass

import numpy as np
import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "sorernn_amd", "csrc")
C = 64  # chunk length


@dataclass
class Shape:
    name: str
    B: int
    T: int
    H: int
    HV: int
    K: int
    V: int
    cu: tuple[int, ...] | None = None

    @property
    def N(self) -> int:
        return len(self.cu) - 1 if self.cu else self.B

    def seqs(self):
        """(n, bos, eos, chunk_first) of every sequence, in token coordinates of the flat [B*T] axis."""
        out, first = [], 0
        for n in range(self.N):
            bos, eos = (self.cu[n], self.cu[n + 1]) if self.cu else (n * self.T, (n + 1) * self.T)
            out.append((n, bos, eos, first))
            first += -(-(eos - bos) // C)
        return out

    @property
    def chunks(self) -> int:
        return sum(-(-(e - b) // C) for _, b, e, _ in self.seqs())

    @property
    def tokens(self) -> int:
        return self.B * self.T


def _cu(lengths):
    return tuple(int(x) for x in np.concatenate([[0], np.cumsum(lengths)]))


def _config3_lengths():
    rng = np.random.default_rng(1003)
    raw = rng.integers(512, 8193, size=8).astype(np.float64)
    lens = np.floor(raw / raw.sum() * 32768).astype(np.int64)
    lens[-1] += 32768 - lens.sum()
    return lens


SHAPES = [
    Shape("config1", 4, 4096, 16, 16, 128, 128),
    Shape("config3", 1, 32768, 16, 16, 128, 128, _cu(_config3_lengths())),
    Shape("config4", 2, 8192, 16, 16, 128, 128),
    Shape("ragged_gva2_d64", 3, 200, 2, 4, 64, 64),
    Shape("varlen_short_docs", 1, 326, 2, 4, 128, 64, _cu([1, 2, 1, 64, 65, 3, 127, 63])),
    Shape("varlen_k64_v128", 1, 257, 4, 4, 64, 128, _cu([100, 157])),
]
GATE_BYTES = [(4, 4), (2, 2), (2, 4), (4, 2)]  # (g, beta) element bytes: fp32 or bf16


class OutOfBounds(AssertionError):
    pass


def check(label, tensor_bytes, base, nrec, off, width):
    """Every access whose first byte lies inside its resource [base, base + nrec) must lie inside the
    tensor [0, tensor_bytes). Arrays broadcast; returns the number of executed accesses."""
    base, nrec, off = np.broadcast_arrays(np.asarray(base, np.int64), np.asarray(nrec, np.int64),
                                          np.asarray(off, np.int64))
    run = off < nrec
    lo = base + off
    bad = run & ((lo < 0) | (lo + width > tensor_bytes))
    if bad.any():
        i = np.argwhere(bad)[0]
        raise OutOfBounds(f"{label}: access at byte {int(lo[tuple(i)])} width {width} outside "
                          f"[0, {tensor_bytes}) (index {tuple(int(x) for x in i)})")
    return int(run.sum())


def check_plain(label, tensor_bytes, byte_off, width, active=True):
    """A plain (non-buffer) access executed where `active` holds."""
    byte_off, active = np.broadcast_arrays(np.asarray(byte_off, np.int64), np.asarray(active, bool))
    bad = active & ((byte_off < 0) | (byte_off + width > tensor_bytes))
    if bad.any():
        i = np.argwhere(bad)[0]
        raise OutOfBounds(f"{label}: plain access at byte {int(byte_off[tuple(i)])} width {width} outside "
                          f"[0, {tensor_bytes})")
    return int(active.sum())


def chunk_rows(s: Shape, extra: int = 0):
    """Per (sequence, chunk c < nc + extra): c0, len (0 for c >= nc), global chunk index, sequence n."""
    c0, ln, cg, nn = [], [], [], []
    for n, bos, eos, first in s.seqs():
        nc = -(-(eos - bos) // C)
        for c in range(nc + extra):
            start = bos + C * c
            c0.append(start)
            ln.append(max(0, min(C, eos - start)) if c < nc else 0)
            cg.append(first + c)
            nn.append(n)
    return (np.array(c0, np.int64), np.array(ln, np.int64), np.array(cg, np.int64), np.array(nn, np.int64))


def _col(x):
    return np.asarray(x, np.int64)[:, None, None]


def _mid(x):
    return np.asarray(x, np.int64)[None, :, None]


def _last(x):
    return np.asarray(x, np.int64)[None, None, :]


# ---------------------------------------------------------------- gate loads
def gate_loads(s: Shape, eg: int, eb: int, extra: int, old_scheme: bool = False) -> int:
    """Gate/beta loads of one wave (lane = token) per (chunk, value head).

    Current state kernel (gdn_chunk.hip::fetch_gates): one 32-bit and one 16-bit load per tensor,
    each through its own resource from the head's element of the chunk's first token; the resource of
    the dtype's width spans (len - 1) * HV * e + e bytes, the other 0 bytes.
    Backward (gdn_chunk_bwd.hip::fetch_gates_bwd): one load of the dtype's width through a resource
    of len * HV * e bytes.
    old_scheme: the state kernel before the fix -- both widths through one resource of len * HV * e.
    """
    c0, ln, _, _ = chunk_rows(s, extra)
    hv, lane = np.arange(s.HV), np.arange(C)
    done = 0
    for tensor, e in (("g", eg), ("beta", eb)):
        nbytes = s.tokens * s.HV * e
        row = s.HV * e
        base = (_col(c0) * s.HV + _mid(hv)) * e
        off = _last(lane) * row
        if old_scheme:
            for width in (4, 2):
                done += check(f"{tensor} b{8 * width} (old)", nbytes, base, _col(ln) * row, off, width)
        else:
            ext = np.where(ln > 0, (ln - 1) * row + e, 0)
            for width in (4, 2):
                nrec = ext if e == width else np.zeros_like(ext)
                done += check(f"{tensor} b{8 * width}", nbytes, base, _col(nrec), off, width)
    return done


def gate_loads_bwd(s: Shape, eg: int, eb: int) -> int:
    c0, ln, _, _ = chunk_rows(s)
    hv, lane = np.arange(s.HV), np.arange(C)
    done = 0
    for tensor, e in (("g", eg), ("beta", eb)):
        base = (_col(c0) * s.HV + _mid(hv)) * e
        done += check(f"bwd {tensor}", s.tokens * s.HV * e, base, _col(ln) * s.HV * e, _last(lane) * s.HV * e, e)
    return done


# ---------------------------------------------------------------- forward state kernel
def state_kernel_grid(s: Shape):
    """Workgroup -> (chain rank, V-slice), gdn_chunk.hip: blockIdx b on XCD b % 8, all slices of a
    chain on one XCD when the chain count is a multiple of 8. Returns (rank, vb) per workgroup."""
    nvb = s.V // 32
    chains = s.N * s.HV
    b = np.arange(chains * nvb)
    if chains % 8 == 0:
        x, j = b % 8, b // 8
        return 8 * (j // nvb) + x, j % nvb
    return b // nvb, b % nvb


def state_kernel(s: Shape, eg: int, eb: int, save: bool) -> int:
    K, V, H, HV = s.K, s.V, s.H, s.HV
    rep = HV // H
    kch = K // 8
    qkpt = C * kch // 256
    done = 0
    # q/k rows of chunks c < nc + 3 (fetch_rows, one step ahead of the staging: thread tq of the q/k
    # waves, 16-byte piece tq % KCH of rows tq / KCH + (256 / KCH) u)
    c0, ln, cg, nn = chunk_rows(s, extra=3)
    h = np.arange(H)
    qk_row = H * K * 2
    tq = np.arange(256)
    off = ((tq // kch) * qk_row + (tq % kch) * 16)[:, None] + (np.arange(qkpt) * (256 // kch) * qk_row)[None, :]
    base = (_col(c0) * H + _mid(h)) * K * 2
    for name in ("q", "k"):
        done += check(f"fwd {name} rows", s.tokens * H * K * 2, base, _col(ln) * qk_row, _last(off.ravel()), 16)
    # T - I rows and the V slice of chunks c < nc + 2 (fetch_tv, one step ahead of the staging:
    # threads tq < 128 of waves 4, 5)
    c0, ln, cg, nn = chunk_rows(s, extra=2)
    t_row, v_row = HV * C * 2, HV * V * 2
    tq = np.arange(128)
    off_t = ((tq >> 3) * t_row + (tq & 7) * 16)[:, None] + (np.arange(4) * 16 * t_row)[None, :]
    tw_bytes = -(-(s.tokens * HV * C * 2) // 256) * 256
    hv = np.arange(HV)
    done += check("fwd T-I rows", tw_bytes, (_col(c0) * HV + _mid(hv)) * C * 2, _col(ln) * t_row,
                  _last(off_t.ravel()), 16)
    off_v = ((tq >> 2) * v_row + (tq & 3) * 16)[:, None] + (np.arange(2) * 32 * v_row)[None, :]
    for vb in range(V // 32):
        base_v = ((_col(c0) * HV + _mid(hv)) * V + vb * 32) * 2
        done += check(f"fwd v slice {vb}", s.tokens * HV * V * 2, base_v, _col(ln) * v_row, _last(off_v.ravel()), 16)
    # gates of chunks c < nc + 3 (two steps ahead of the staging, one more in flight)
    done += gate_loads(s, eg, eb, extra=3)
    # O stores of chunks c < nc (store_o: the V-slice layout)
    c0, ln, cg, nn = chunk_rows(s)
    for vb in range(V // 32):
        base_o = ((_col(c0) * HV + _mid(hv)) * V + vb * 32) * 2
        done += check(f"fwd o slice {vb}", s.tokens * HV * V * 2, base_o, _col(ln) * v_row, _last(off_v.ravel()), 16)
    # the fused norm's progress words, NVB per chain (4 bytes each) at the start of the chain's
    # 64-word block: a slice stores its own word through a resource over its chain's words
    # (publish_o); an epilogue wave polls them with lane l reading word l (lanes l >= NVB fall
    # outside the resource)
    nvb, chains, stride = V // 32, s.N * HV, 64
    base_w, nrec_w = _col(np.arange(chains) * stride * 4), _col(np.full(chains, nvb * 4))
    done += check("fwd norm progress store", chains * stride * 4, base_w, nrec_w, _last(np.arange(nvb) * 4), 4)
    done += check("fwd norm progress poll", chains * stride * 4, base_w, nrec_w, _last(np.arange(64) * 4), 4)
    # the epilogue workgroups' XCC posts (word 16 + r of the chain's whole 64-word block, r < 48) and
    # the slices' reads of them (lane l reads word 16 + l; lanes past the block read nothing)
    nrec_b = _col(np.full(chains, stride * 4))
    done += check("fwd norm epilogue post", chains * stride * 4, base_w, nrec_b, _last((16 + np.arange(48)) * 4), 4)
    done += check("fwd norm post read", chains * stride * 4, base_w, nrec_b, _last((16 + np.arange(64)) * 4), 4)
    # the epilogue's O loads, gate loads and y stores (norm_epilogue): per (chunk, head) a resource
    # over the chunk's valid rows of the head, offsets row * HV * V * 2 + 16-byte piece for the
    # 64 rows of the tile and V / 8 pieces per row
    off_e = (np.arange(C)[:, None] * v_row + (np.arange(V // 8) * 16)[None, :]).ravel()
    base_e = (_col(c0) * HV + _mid(hv)) * V * 2
    for name in ("o", "gate"):
        done += check(f"fwd norm epilogue {name}", s.tokens * HV * V * 2, base_e, _col(ln) * v_row, _last(off_e), 16)
    # h0 loads / ht stores (plain, fp32 [N][HV][K][V]) and, with SAVE, the state entering each chunk
    # (bf16 [chunks][HV][V][K], an 8-byte store per lane and state tile)
    rank, vbs = state_kernel_grid(s)
    assert sorted(zip(rank.tolist(), vbs.tolist())) == [(r, v) for r in range(s.N * HV) for v in range(V // 32)], \
        "state-kernel workgroups must cover every (chain, V-slice) exactly once"
    kt = K // 16
    a = np.arange(kt)
    lane = np.arange(64)
    g4, li = lane >> 4, lane & 15
    kd0 = (32 * (a >> 1))[:, None] + (8 * g4)[None, :] + (4 * (a & 1))[:, None]          # [a, lane]
    key = kd0[:, :, None] + np.arange(4)[None, None, :]                                   # [a, lane, r]
    for sw in (0, 1):
        col = (vbs * 32 + 16 * sw)[:, None, None, None] + li[None, None, :, None]        # [wg, 1, lane, 1]
        idx = (rank[:, None, None, None] * K + key[None]) * V + col                      # chain = n * HV + hv
        done += check_plain("fwd h0/ht", s.N * HV * K * V * 4, idx * 4, 4)
    if save:
        chunks = s.chunks
        rank_hv = rank % HV
        rank_n = rank // HV  # identity order (the longest-first order is a permutation of sequences)
        first = np.array([f for _, _, _, f in s.seqs()], np.int64)
        ncs = np.array([-(-(e - b) // C) for _, b, e, _ in s.seqs()], np.int64)
        ls = np.arange(64)
        for sw in (0, 1):
            lane_off = (((vbs[:, None] * 32 + 16 * sw + (ls & 15)[None, :]) * K + 8 * (ls >> 4)[None, :]) * 2)
            tile_off = (32 * (a >> 1) + 4 * (a & 1)) * 2
            off = lane_off[:, :, None] + tile_off[None, None, :]                           # [wg, lane, a]
            for c in range(int(ncs.max())):
                live = c < ncs[rank_n]
                base = ((first[rank_n] + c) * HV + rank_hv) * K * V * 2
                nrec = np.where(live, K * V * 2, 0)
                done += check("fwd saved state", chunks * HV * V * K * 2, base[:, None, None], nrec[:, None, None],
                              off, 8)
    _ = rep
    return done


def prep_kernel(s: Shape, eg: int, eb: int) -> int:
    """gdn_chunk_prep.hip. The one-wave kernel loads the k rows of a chunk through a resource over
    its valid rows of head h (lane offsets row * H * K * 2 + 16-byte piece, every row of the tile);
    the workgroup kernel kept for comparison loads them plainly, guarded by row < len. Both load the
    gates plainly (lane = token < len) and store the T - I rows as plain 16-byte stores guarded by
    row < len."""
    c0, ln, _, _ = chunk_rows(s)
    K, H, HV = s.K, s.H, s.HV
    kch = K // 8
    e = np.arange(C * kch)
    row, c8 = e // kch, e % kch
    done = 0
    off = row * H * K * 2 + c8 * 16
    done += check("prep k (resource)", s.tokens * H * K * 2, (_col(c0) * H + _mid(np.arange(H))) * K * 2,
                  _col(ln) * H * K * 2, _last(off), 16)
    for hv in range(HV):
        h = hv // (HV // H)
        idx = ((_col(c0)[:, :, 0] + row[None, :]) * H + h) * K + c8[None, :] * 8
        done += check_plain("prep k", s.tokens * H * K * 2, idx * 2, 16, row[None, :] < ln[:, None])
        gi = (c0[:, None] + np.arange(C)[None, :]) * HV + hv
        live = np.arange(C)[None, :] < ln[:, None]
        done += check_plain("prep g", s.tokens * HV * eg, gi * eg, eg, live)
        done += check_plain("prep beta", s.tokens * HV * eb, gi * eb, eb, live)
        e8 = np.arange(C * 8)
        r8, p8 = e8 >> 3, e8 & 7
        ti = ((c0[:, None] + r8[None, :]) * HV + hv) * C + p8[None, :] * 8
        tw_bytes = -(-(s.tokens * HV * C * 2) // 256) * 256
        done += check_plain("prep T-I store", tw_bytes, ti * 2, 16, r8[None, :] < ln[:, None])
    return done


# ---------------------------------------------------------------- backward
def _qk_rows(label, s, c0, ln, nt):
    """fetch_qk<KD, NT>: thread tid < NT, row tid / KCH + u RPP, piece tid % KCH."""
    kch = s.K // 8
    rpp = nt // kch
    tid = np.arange(nt)
    off = ((tid // kch)[:, None] + (np.arange(C // rpp) * rpp)[None, :]) * (s.H * s.K * 2) + ((tid % kch) * 16)[:, None]
    base = (_col(c0) * s.H + _mid(np.arange(s.H))) * s.K * 2
    return check(label, s.tokens * s.H * s.K * 2, base, _col(ln) * s.H * s.K * 2, _last(off.ravel()), 16)


def _slice(label, tensor_bytes, base, ln, rb, w16, nt):
    """fetch_slice<W, NT>: piece e = u NT + tid, row e / (W/8), 16-byte piece e % (W/8) of a row of
    rb bytes; base [chunk, head] in bytes."""
    ch = w16 // 8
    e = np.arange(C * ch)
    off = (e // ch) * rb + (e % ch) * 16
    assert C * ch % nt == 0
    return check(label, tensor_bytes, base[:, :, None], _col(ln) * rb, _last(off), 16)


def bwd_kernels(s: Shape, eg: int, eb: int) -> int:
    K, V, H, HV = s.K, s.V, s.H, s.HV
    c0, ln, cg, nn = chunk_rows(s)
    hv = np.arange(HV)
    v_row, t_row = HV * V * 2, HV * C * 2
    tok_v, tw_bytes = s.tokens * HV * V * 2, -(-(s.tokens * HV * C * 2) // 256) * 256
    tn_bytes = s.tokens * HV * C * 2
    g1_bytes = s.chunks * HV * V * C * 2  # bf16 [chunks][HV][V][64 tokens]
    done = 0
    # 1. prep kernel (per chunk, value head)
    done += _qk_rows("bwd prep k", s, c0, ln, 256) + _qk_rows("bwd prep q", s, c0, ln, 256)
    done += _slice("bwd prep dO", tok_v, (c0[:, None] * HV + hv[None, :]) * V * 2, ln, v_row, V, 256)
    done += _slice("bwd prep T-I", tw_bytes, (c0[:, None] * HV + hv[None, :]) * C * 2, ln, t_row, C, 256)
    done += gate_loads_bwd(s, eg, eb)
    e = np.arange(2 * 256)
    row, j0 = e >> 3, (e & 7) * 8
    live = row[None, None, :] < ln[:, None, None]
    tnt = ((c0[:, None, None] + row[None, None, :]) * HV + hv[None, :, None]) * C + j0[None, None, :]
    done += check_plain("bwd prep (T-I)^T store", tn_bytes, tnt * 2, 16, live)
    # G1: wave w, lane (g, i) stores tokens 16w + 4g..+3 of column 16ct + i, every chunk slot
    ct = np.arange(V // 16)
    col = (16 * ct[:, None] + np.arange(16)[None, :]).ravel()
    tt = (16 * np.arange(4)[:, None] + 4 * np.arange(4)[None, :]).ravel()
    g1i = ((cg[:, None, None, None] * HV + hv[None, :, None, None]) * V + col[None, None, :, None]) * C + \
        tt[None, None, None, :]
    done += check_plain("bwd prep G1 store", g1_bytes, g1i * 2, 8)
    # 2. reverse state kernel (per sequence, value head, 32 value columns; chunks from last to first)
    done += _qk_rows("bwd state k", s, c0, ln, 128) + _qk_rows("bwd state q", s, c0, ln, 128)
    done += _slice("bwd state (T-I)^T", tn_bytes, (c0[:, None] * HV + hv[None, :]) * C * 2, ln, t_row, C, 128)
    for vb in range(V // 32):
        done += _slice(f"bwd state dO {vb}", tok_v, ((c0[:, None] * HV + hv[None, :]) * V + vb * 32) * 2, ln, v_row,
                       32, 128)
        g1s = ((cg[:, None, None] * HV + hv[None, :, None]) * V + vb * 32) * C * 2 + 16 * np.arange(256)[None, None, :]
        done += check_plain(f"bwd state G1 {vb}", g1_bytes, g1s, 16)
    lane = np.arange(64)
    g4, li = lane >> 4, lane & 15
    kt = np.arange(K // 16)
    for vb in range(V // 32):
        for sw in (0, 1):
            col = vb * 32 + 16 * sw + li
            dp = (((cg[:, None, None] * HV + hv[None, :, None]) * V + col[None, None, :]) * K + 4 * g4[None, None, :])
            done += check_plain("bwd state dS' store", s.chunks * HV * V * K * 2,
                                (dp[..., None] + 16 * kt) * 2, 8)
            for n in range(s.N):
                key = 16 * kt[:, None, None] + 4 * g4[None, :, None] + np.arange(4)[None, None, :]
                idx = ((n * HV + hv[:, None, None, None]) * K + key[None]) * V + col[None, None, :, None]
                done += check_plain("bwd dht/dh0", s.N * HV * K * V * 4, idx * 4, 4)
    # 3. gradient kernel (per chunk, q/k head; the value heads of the group in turn, V in 32-column passes)
    done += _qk_rows("bwd grad k", s, c0, ln, 256) + _qk_rows("bwd grad q", s, c0, ln, 256)
    t = np.arange(256)
    w = t >> 6
    tok0 = 16 * w
    lq = t & 63
    nsp = K // 64
    for pi in range(V // 32):
        hs_off = (((cg[:, None, None] * HV + hv[None, :, None]) * V + 32 * pi) * K +
                  (np.arange(nsp)[:, None] * 256 + t[None, :]).ravel()[None, None, :] * 8)
        done += check_plain("bwd grad S^T / dS'^T rows", s.chunks * HV * V * K * 2, hs_off * 2, 16)
        row, chq = t >> 2, t & 3
        for label, nbytes in (("bwd grad dO pass", tok_v), ("bwd grad V pass", tok_v)):
            done += check(label, nbytes, ((_col(c0) * HV + _mid(hv)) * V + 32 * pi) * 2, _col(ln) * v_row,
                          _last(row * v_row + chq * 16), 16)
        g_off = ((32 * pi + 16 * np.arange(2)[None, :] + (t & 15)[:, None]) * C + (tok0 + 4 * ((t & 63) >> 4))[:, None])
        done += check_plain("bwd grad G1 pass", g1_bytes,
                            ((cg[:, None, None] * HV + hv[None, :, None]) * V * C + g_off.ravel()[None, None, :]) * 2, 8)
        tf_off = ((tok0 + (lq & 15))[:, None] * t_row + (32 * np.arange(2)[None, :] + 8 * (lq >> 4)[:, None]) * 2).ravel()
        # the forward's fp16 T - I rows (piece 4u + g at the same byte offset) and the (T - I)^T rows
        for label, nbytes in (("bwd grad T-I rows (forward's fp16)", tw_bytes), ("bwd grad (T-I)^T rows", tn_bytes)):
            done += check(label, nbytes, (_col(c0) * HV + _mid(hv)) * C * 2, _col(ln) * t_row, _last(tf_off), 16)
    kch = K // 8
    rpp = 256 // kch
    raw_off = ((t // kch)[:, None] + (np.arange(C // rpp) * rpp)[None, :]) * (H * K * 2) + ((t % kch) * 16)[:, None]
    for name in ("q", "k"):
        done += check(f"bwd grad raw {name} (l2 backward)", s.tokens * H * K * 2,
                      (_col(c0) * H + _mid(np.arange(H))) * K * 2, _col(ln) * H * K * 2, _last(raw_off.ravel()), 16)
    return done


# ---------------------------------------------------------------- tests
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s.name)
@pytest.mark.parametrize("eg,eb", GATE_BYTES, ids=lambda x: f"{x}")
def test_forward_state_kernel_stays_inside_its_tensors(shape, eg, eb):
    assert state_kernel(shape, eg, eb, save=shape.name not in ("config3",)) > 0


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s.name)
def test_prep_kernel_stays_inside_its_tensors(shape):
    for eg, eb in ((4, 4), (2, 2)):
        assert prep_kernel(shape, eg, eb) > 0


@pytest.mark.parametrize("shape", [s for s in SHAPES if s.name != "config3"], ids=lambda s: s.name)
@pytest.mark.parametrize("eg,eb", [(4, 4), (2, 2)], ids=lambda x: f"{x}")
def test_backward_kernels_stay_inside_their_tensors(shape, eg, eb):
    assert bwd_kernels(shape, eg, eb) > 0


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s.name)
def test_checker_flags_the_old_gate_loads(shape):
    """The pre-fix loads read past a 16-bit gate tensor (the last head's last token); fp32 was safe."""
    with pytest.raises(OutOfBounds, match=r"g b32 \(old\).*width 4"):
        gate_loads(shape, 2, 2, extra=3, old_scheme=True)
    assert gate_loads(shape, 4, 4, extra=3, old_scheme=True) > 0
    # the byte the old scheme touched at config 1: the bf16 tensor is 524,288 B, its last load ends at 524,290
    if shape.name == "config1":
        last = ((shape.tokens - 1) * shape.HV + shape.HV - 1) * 2
        assert last + 4 == shape.tokens * shape.HV * 2 + 2 == 524_290


def test_model_covers_every_buffer_resource():
    """Each buffer resource a kernel file creates has a counterpart above; a new one must be modelled."""
    expected = {"gdn_chunk.hip": 15, "gdn_chunk_bwd.hip": 9, "gdn_chunk_prep.hip": 1}
    for fname, n in expected.items():
        with open(os.path.join(CSRC, fname)) as f:
            src = f.read()
        assert len(re.findall(r"\bmake_rsrc\(", src)) == n, fname
