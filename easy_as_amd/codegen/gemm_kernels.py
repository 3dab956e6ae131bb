"""gfx950 MFMA GEMM emitted for kernels that ``gemm_lift`` proved to be dense GEMMs.

Launches of more than 128 rows tile C into 256 x 256 workgroup tiles (or 128 x
128, below; the fp32 templates at the end of this module use 64 x 64 and 128 x 128).
The 16-bit source is written once for its MFMA operand type ``eas_op_t``: f16, or
bf16 when the kernel's threadgroup tiles are bf16 (``_OP_TYPES`` supplies the type,
the MFMA and the transposing LDS read; everything else is the same).  It has these
entry points, and the launch plan (``gemm_lift.plan_gemm``) picks one:

* ``<name>__pp`` (512 threads): the 8-wave ping-pong DMA body for A and B of the
  operand type whose rows the DMA takes.  Waves w and w+4 share a SIMD; the two groups of
  four waves alternate load phases and MFMA phases one barrier apart, each
  wave holding 128 x 64 of the tile (8 x 4 ``v_mfma_f32_16x16x32_f16``
  accumulators; ``EAS_HIP_GEMM_MFMA=32`` selects 4 x 2 of ``32x32x16``).
* ``<name>__t128``, ``<name>__t128x256``, ``<name>__t64x64`` and ``<name>__t128x64``
  (512 threads): the same DMA operands on 128 x 128, 128 x 256, 64 x 64 and
  128 x 64 tiles, for launches whose 256 x 256 grid would leave CUs idle: 4 waves
  issue the DMA, 4 waves of 64 x 64 (64 x 128, 32 x 32, 64 x 32) read fragments
  and run the MFMAs.
* ``<name>`` (256 threads, 4 waves of 128 x 128, 4 x 4 accumulators in 256
  AGPRs): the skinny path (launches of at most 128 rows), the 4-wave DMA body,
  and the register body; a uniform branch picks one per launch.

DMA bodies (A and B of the operand type; K and ldb even and 4-byte aligned bases, so every row
is 4-byte aligned; each matrix under 2 GiB):

* A and B go HBM -> LDS with ``buffer_load_dwordx4 ... lds`` (no staging
  registers), BK = 32 per stage, a 4-stage ring (128 KB), so loads are issued
  three stages ahead;
* LDS holds A as [m][k] and B as [k][n] (the layouts of HBM); 16-byte chunks
  are XOR-swizzled by row so fragment reads are bank-conflict free;
* A fragments are ``ds_read_b128`` (8 consecutive k per lane); B fragments are
  two ``ds_read_b64_tr_b16`` per MFMA operand, which transpose a 4(k) x 16(n)
  block across each 16-lane group so every lane receives k-contiguous B;
* buffer range checks (per dword) give zeros for rows past M and for B rows
  past K; the lanes of the K tail stage that would read past K in A use an
  offset outside the range, and when K is not a multiple of 8 the halves of
  the last chunk of each row that lie past K are zeroed (the 4-wave body in
  LDS once the tail stage has landed, the 8-wave body in its A fragments);
* the 4-wave iteration is scheduled by hand (``sched_barrier``): ks0 MFMAs
  overlap the ks1 fragment reads; after the mid-iteration barrier the ks1
  MFMAs overlap the DMA issue (one every two MFMAs) and the next stage's ks0
  fragment reads.

Register body (any other case, including f32 inputs that MFMA consumes as f16):
global -> registers -> LDS, BK = 64, double buffered; A loads use the widest
vector (up to 16 bytes) that K's row alignment allows; B is transposed in
registers (each thread loads an 8(k) x 8(n) block) so LDS holds B as [n][k];
edge tiles and the K tail load element by element with zero fill straight into
LDS.

Tile order is XCD aware: workgroup w runs on XCD w % 8, so each XCD gets a
contiguous range of tiles, grouped 4 tile-rows high for L2 reuse.

The kernel computes C[m, n] for m in [m_lo, m_hi), n in [n_lo, n_hi) (hidden
arguments: the rectangle the reference launch covers); it moves its base
pointers to (m_lo, n_lo) on entry, so every body works on a sub-matrix whose
origin is 0.  Rows of A have length K (a compile-time constant); B and C rows
have the scalar argument ``ldb`` as stride.  B's buffer range is the extent the
rectangle is proven to read, (K-1)*ldb + N, so tile-wide reads past it return 0.
"""

from __future__ import annotations

import os

from ..ir import DType, IRModule
from .gemm_lift import GemmSpec
from .hip import PRELUDE, Geometry, Lowered, ctype

_DMA_HELPERS = r"""
typedef float eas_f32x16 __attribute__((ext_vector_type(16)));
typedef int eas_rsrc __attribute__((ext_vector_type(4)));
#define EAS_LDS __attribute__((address_space(3)))
// s_waitcnt with only vmcnt limited (gfx9 encoding: vmcnt[3:0], [15:14]; expcnt and lgkmcnt at max)
#define EAS_WAITVM(n) (((n) & 15) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
// s_waitcnt lgkmcnt(0) with vmcnt and expcnt at max
#define EAS_WAITLGKM0 (15 | (3 << 14) | (0x7 << 4))

// raw buffer resource: base, range in bytes (reads at or past it return 0), gfx9 word 3
static __device__ __forceinline__ eas_rsrc eas_make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  eas_rsrc r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xffffu);
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}
// 16 bytes per lane, HBM -> LDS; lane i writes LDS bytes [lds + 16 i, lds + 16 i + 16).
// Issued as asm so the compiler does not add vmcnt(0) before every LDS read; the
// pipelines count their own loads with EAS_WAITVM.
static __device__ __forceinline__ void eas_dma16(eas_rsrc r, uint32_t voff, uint32_t lds) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}
// The same with the stage part of the offset in an SGPR (soffset): the lane part stays fixed in
// one VGPR per load, so a wave that only issues these runs no VALU.  Every caller keeps
// voff + soff inside the buffer, or voff at 2^31 or more with soff below 2^31 (zeros), so the
// result does not depend on whether the range check includes soffset.
static __device__ __forceinline__ void eas_dma16s(eas_rsrc r, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(lds) : "memory");
}
"""

# The MFMA operand type of the 16-bit templates: f16 or bf16 (the dtype of the kernel's
# threadgroup tiles).  Both have 16-bit elements, so the DMA, LDS layout and transposed
# reads are the same; only the element type, the MFMA and the transposing read differ.
_OP_TYPES = {
    DType.F16: r"""
typedef _Float16 eas_op_t;
typedef __fp16 eas_h4t __attribute__((__vector_size__(4 * sizeof(__fp16))));
#define EAS_MFMA32 __builtin_amdgcn_mfma_f32_32x32x16_f16
#define EAS_MFMA16 __builtin_amdgcn_mfma_f32_16x16x32_f16
#define EAS_DS_TR16 __builtin_amdgcn_ds_read_tr16_b64_v4f16
""",
    DType.BF16: r"""
typedef __bf16 eas_op_t;
typedef __bf16 eas_h4t __attribute__((ext_vector_type(4)));
#define EAS_MFMA32 __builtin_amdgcn_mfma_f32_32x32x16_bf16
#define EAS_MFMA16 __builtin_amdgcn_mfma_f32_16x16x32_bf16
#define EAS_DS_TR16 __builtin_amdgcn_ds_read_tr16_b64_v4bf16
""",
}

_TEMPLATE = r"""
typedef eas_op_t eas_h8 __attribute__((ext_vector_type(8)));
typedef eas_op_t eas_h4 __attribute__((ext_vector_type(4)));

template <typename T> static __device__ __forceinline__ eas_h8 eas_load8(const T* p);
template <> __device__ __forceinline__ eas_h8 eas_load8<eas_op_t>(const eas_op_t* p) { return *(const eas_h8*)p; }
template <> __device__ __forceinline__ eas_h8 eas_load8<float>(const float* p) {
  const eas_f32x4 lo = *(const eas_f32x4*)p, hi = *(const eas_f32x4*)(p + 4);
  eas_h8 v;
  v[0] = (eas_op_t)lo[0]; v[1] = (eas_op_t)lo[1]; v[2] = (eas_op_t)lo[2]; v[3] = (eas_op_t)lo[3];
  v[4] = (eas_op_t)hi[0]; v[5] = (eas_op_t)hi[1]; v[6] = (eas_op_t)hi[2]; v[7] = (eas_op_t)hi[3];
  return v;
}

// elements per load for rows of `k` elements of T: the widest power of two up to 16 bytes dividing k
template <typename T> constexpr int eas_row_vec(int k) {
  int v = 16 / (int)sizeof(T);
  while (v > 1 && k % v != 0) v /= 2;
  return v;
}
// 8 consecutive elements from rows whose alignment allows AL-element vector loads
template <typename T, int AL> static __device__ __forceinline__ eas_h8 eas_load8_al(const T* p) {
  if constexpr (AL >= 8 && sizeof(T) == 2) {
    return *(const eas_h8*)p;
  } else if constexpr (AL == 1) {
    eas_h8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (eas_op_t)p[e];
    return v;
  } else {
    constexpr int W = AL > 8 ? 8 : AL;
    typedef T vec_t __attribute__((ext_vector_type(W)));
    eas_h8 v;
#pragma unroll
    for (int e = 0; e < 8; e += W) {
      const vec_t x = *(const vec_t*)(p + e);
#pragma unroll
      for (int i = 0; i < W; ++i) v[e + i] = (eas_op_t)x[i];
    }
    return v;
  }
}

template <typename CT, int K>
static __device__ __forceinline__ void eas_gemm_dma(const eas_op_t* __restrict__ A, const eas_op_t* __restrict__ B,
                                                    CT* __restrict__ C, int ldb, int M, int N, int m0, int n0,
                                                    eas_op_t* smem) {
  constexpr int BM = 256, BN = 256, BK = 32, NSTAGE = 4, KT = (K + BK - 1) / BK;
  constexpr int STAGE_H = BM * BK;  // halves per operand per stage (16 KB)
  eas_op_t* As = smem;
  eas_op_t* Bs = smem + NSTAGE * STAGE_H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const eas_rsrc ra = eas_make_rsrc(A, (uint32_t)M * (uint32_t)K * 2u);
  const eas_rsrc rb = eas_make_rsrc(B, ((uint32_t)(K - 1) * (uint32_t)ldb + (uint32_t)N) * 2u);
  // DMA instruction q = 4 wave + i writes 1 KB of a stage.  A: rows 16q + lane/4, chunk lane%4
  // stored at chunk ^ ((row/4)%4).  B: rows (k) 2q + lane/32, chunk lane%32 stored at chunk ^ 4(row%4).
  uint32_t a_off[4], b_off[4];
  int a_k[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = wave * 4 + i;
    const int r_a = 16 * q + (lane >> 2);
    const int c_a = (lane & 3) ^ ((r_a >> 2) & 3);
    a_off[i] = ((uint32_t)(m0 + r_a) * (uint32_t)K + (uint32_t)(c_a * 8)) * 2u;
    a_k[i] = c_a * 8;
    const int r_b = 2 * q + (lane >> 5);
    const int c_b = (lane & 31) ^ (4 * (r_b & 3));
    b_off[i] = ((uint32_t)r_b * (uint32_t)ldb + (uint32_t)(n0 + c_b * 8)) * 2u;
  }
  const uint32_t lds_a = (uint32_t)(size_t)(EAS_LDS eas_op_t*)As, lds_b = (uint32_t)(size_t)(EAS_LDS eas_op_t*)Bs;
  auto dma_one = [&](int kt, int d) {  // d in 0..7: 0..3 A, 4..7 B
    const int s = kt % NSTAGE, i = d & 3;
    const uint32_t dst = (uint32_t)((s * STAGE_H + (wave * 4 + i) * 512) * 2);
    if (d < 4) {
      uint32_t off = a_off[i] + (uint32_t)(kt * BK * 2);
      if (K % BK != 0 && kt * BK + a_k[i] >= K) off = 0x80000000u;  // K tail: past the range -> zeros
      eas_dma16(ra, off, lds_a + dst);
    } else {
      uint32_t off = b_off[i] + (uint32_t)kt * (uint32_t)(BK * 2) * (uint32_t)ldb;
      if (K % BK != 0 && kt * BK + 2 * (wave * 4 + i) + (lane >> 5) >= K) off = 0x80000000u;  // B rows past K
      eas_dma16(rb, off, lds_b + dst);
    }
  };
  // Rows of A need only 4-byte alignment: a 16-byte DMA chunk may start anywhere, and at the end
  // of a row whose length K is not a multiple of 8 the last chunk runs into the next row.  Once
  // the tail stage has landed, those halves (k >= K) are zeroed in LDS, so a non-finite value in
  // the next row never meets B's zero rows.  One row per thread (BM = 256).
  auto fix_tail = [&]() {
    if constexpr (K % 8 != 0) {
      constexpr int KR = K % BK, CP = KR / 8, E0 = KR % 8;
      const int r = tid;
      eas_op_t* row = As + ((KT - 1) % NSTAGE) * STAGE_H + r * BK + ((CP ^ ((r >> 2) & 3)) * 8);
#pragma unroll
      for (int e = E0; e < 8; ++e) row[e] = (eas_op_t)0.0f;
    }
  };
  // fragment offsets (halves within a stage)
  int fa_off[2][4], fb_off[2][4][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wm * 128 + i * 32 + (lane & 31);
      const int c = (2 * ks + (lane >> 5)) ^ ((r >> 2) & 3);
      fa_off[ks][i] = r * BK + c * 8;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // ds_read_b64_tr_b16: in each 16-lane group, source lane kq addresses row kq/4, columns 4(kq%4)..+3;
        // result lane i receives column i for the four rows
        const int gq = lane >> 4, kq = lane & 15;
        const int row = 16 * ks + 8 * (gq >> 1) + 4 * h + (kq >> 2);
        const int col = wn * 128 + j * 32 + 16 * (gq & 1) + 4 * (kq & 3);
        const int chunk = (col >> 3) ^ (4 * (row & 3));
        fb_off[ks][j][h] = row * BN + chunk * 8 + (col & 7);
      }
  }
  eas_h8 fa[2][4], fb[2][4];
  auto read_a = [&](int s, int ks, int i) { fa[ks][i] = *(const eas_h8*)(As + s * STAGE_H + fa_off[ks][i]); };
  auto read_b = [&](int s, int ks, int j) {
    const eas_op_t* bs = Bs + s * STAGE_H;
    const eas_h4t lo = EAS_DS_TR16((EAS_LDS eas_h4t*)(bs + fb_off[ks][j][0]));
    const eas_h4t hi = EAS_DS_TR16((EAS_LDS eas_h4t*)(bs + fb_off[ks][j][1]));
    const eas_h4 l4 = __builtin_bit_cast(eas_h4, lo), h4 = __builtin_bit_cast(eas_h4, hi);
    fb[ks][j] = (eas_h8){l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
  };
  eas_f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (eas_f32x16){};
  auto mfma_row = [&](int ks, int i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = EAS_MFMA32(fa[ks][i], fb[ks][j], acc[i][j], 0, 0, 0);
  };
  // this wave's loads of the awaited stage are done; `later` newer stages (8 loads each) may stay in flight
  auto wait_stage = [&](int later) {
    if (later >= 2) __builtin_amdgcn_s_waitcnt(EAS_WAITVM(16));
    else if (later == 1) __builtin_amdgcn_s_waitcnt(EAS_WAITVM(8));
    else __builtin_amdgcn_s_waitcnt(EAS_WAITVM(0));
  };

#pragma unroll
  for (int p = 0; p < NSTAGE - 1; ++p)
    if (p < KT)
#pragma unroll
      for (int d = 0; d < 8; ++d) dma_one(p, d);
  wait_stage(KT - 1 < NSTAGE - 2 ? KT - 1 : NSTAGE - 2);
  __syncthreads();
  if (K % 8 != 0 && KT == 1) {
    fix_tail();
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) { read_b(0, 0, i); read_a(0, 0, i); }
  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt % NSTAGE, sn = (kt + 1) % NSTAGE;
    const bool next = kt + 1 < KT, issue = kt + NSTAGE - 1 < KT;
    // phase A: ks0 MFMAs (set 0) while the ks1 fragments (set 1) load
    __builtin_amdgcn_sched_barrier(0);
    read_b(s, 1, 0); read_b(s, 1, 1);
    mfma_row(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    read_b(s, 1, 2); read_b(s, 1, 3);
    mfma_row(0, 1);
    __builtin_amdgcn_sched_barrier(0);
    read_a(s, 1, 0); read_a(s, 1, 1);
    mfma_row(0, 2);
    __builtin_amdgcn_sched_barrier(0);
    read_a(s, 1, 2); read_a(s, 1, 3);
    mfma_row(0, 3);
    __builtin_amdgcn_sched_barrier(0);
    if (next) {
      // stage kt+1 landed (all waves), and every wave is done with stage kt-1, whose buffer the next DMA refills
      wait_stage(KT - 2 - kt < NSTAGE - 3 ? KT - 2 - kt : NSTAGE - 3);
      __syncthreads();
      if (K % 8 != 0 && kt == KT - 2) {  // the next stage is the tail
        fix_tail();
        __syncthreads();
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // phase B: ks1 MFMAs (set 1); DMA of stage kt+3 and the ks0 fragments of stage kt+1 (set 0)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (issue) dma_one(kt + NSTAGE - 1, 2 * i);
      if (next) read_b(sn, 0, i);
      acc[i][0] = EAS_MFMA32(fa[1][i], fb[1][0], acc[i][0], 0, 0, 0);
      acc[i][1] = EAS_MFMA32(fa[1][i], fb[1][1], acc[i][1], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (issue) dma_one(kt + NSTAGE - 1, 2 * i + 1);
      if (next) read_a(sn, 0, i);
      acc[i][2] = EAS_MFMA32(fa[1][i], fb[1][2], acc[i][2], 0, 0, 0);
      acc[i][3] = EAS_MFMA32(fa[1][i], fb[1][3], acc[i][3], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const bool full = (m0 + BM <= M) && (n0 + BN <= N);
  // lane l, register r of a 32x32 tile holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 128 + i * 32 + (r / 4) * 8 + (lane >> 5) * 4 + (r % 4);
        const int col = n0 + wn * 128 + j * 32 + (lane & 31);
        if (full || (row < M && col < N)) C[(size_t)row * ldb + col] = (CT)acc[i][j][r];
      }
}

// Ping-pong DMA body: 8 waves (two per SIMD; waves w and w+4 share one) in two groups.  Group g
// owns rows [128g, 128g+128) of the 256x256 tile, wave p of the group columns [64p, 64p+64)
// (4 x 2 accumulators of 32x32, 128 registers).  Each wave alternates a load phase (all fragments
// of one BK=32 stage, plus its quarter of the DMA three stages ahead) and an MFMA phase (16 MFMAs),
// separated by workgroup barriers; group 1 enters the loop one barrier later, so while one wave of
// a SIMD runs MFMAs the other one loads.  Stage ring, LDS layout, swizzles and range checks are
// the 4-wave DMA body's.  When K is not a multiple of 8, the A fragments of the tail stage are
// masked to zero past K in registers (the last 16-byte chunk of a row reaches into the next row).
// MI selects the MFMA: 32 (v_mfma_f32_32x32x16: each wave's 128 x 64 as 4 x 2 tiles of 32 x 32,
// two k-steps of 16 per stage) or 16 (v_mfma_f32_16x16x32: 8 x 4 tiles of 16 x 16, one k-step of
// 32 per stage; fewer accumulator bytes move through the MFMA per flop).  Same LDS reads per stage.
template <bool V>
struct eas_bool_c {  // a compile-time flag passed as a value (to select a loop version)
  static constexpr bool value = V;
};
template <typename CT, int K, int MI = 32>
static __device__ __forceinline__ void eas_gemm_pp(const eas_op_t* __restrict__ A, const eas_op_t* __restrict__ B,
                                                   CT* __restrict__ C, int ldb, int M, int N, int m0, int n0,
                                                   eas_op_t* smem) {
  constexpr int BM = 256, BN = 256, BK = 32, NSTAGE = 4, KT = (K + BK - 1) / BK;
  constexpr int STAGE_H = BM * BK;
  eas_op_t* As = smem;
  eas_op_t* Bs = smem + NSTAGE * STAGE_H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave >> 2, p = wave & 3;
  const eas_rsrc ra = eas_make_rsrc(A, (uint32_t)M * (uint32_t)K * 2u);
  const eas_rsrc rb = eas_make_rsrc(B, ((uint32_t)(K - 1) * (uint32_t)ldb + (uint32_t)N) * 2u);
  // DMA instruction q = 2 wave + i writes 1 KB of a stage.  A: rows 16q + lane/4, chunk lane%4
  // stored at chunk ^ ((row/4)%4).  B: rows (k) 2q + lane/32, chunk lane%32 stored at chunk ^ bsw(row):
  // bits 2-3 of the mask spread the four rows of a transposing read over the banks, bit 1 keeps
  // rows 8 apart (the two 16-lane groups of a half-wave in the 16 x 16 x 32 mapping) apart.
  auto bsw = [](int row) { return (4 * (row & 3)) ^ (2 * ((row >> 3) & 1)); };
  uint32_t a_off[2], b_off[2];
  int a_k[2], b_k[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = wave * 2 + i;
    const int r_a = 16 * q + (lane >> 2);
    const int c_a = (lane & 3) ^ ((r_a >> 2) & 3);
    a_off[i] = ((uint32_t)(m0 + r_a) * (uint32_t)K + (uint32_t)(c_a * 8)) * 2u;
    a_k[i] = c_a * 8;
    const int r_b = 2 * q + (lane >> 5);
    const int c_b = (lane & 31) ^ bsw(r_b);
    b_off[i] = ((uint32_t)r_b * (uint32_t)ldb + (uint32_t)(n0 + c_b * 8)) * 2u;
    b_k[i] = r_b;
    // rows past M read zeros through an offset past the range (a row offset could wrap in 32 bits)
    if (m0 + r_a >= M) a_off[i] = 0x80000000u;
  }
  const uint32_t lds_a = (uint32_t)(size_t)(EAS_LDS eas_op_t*)As, lds_b = (uint32_t)(size_t)(EAS_LDS eas_op_t*)Bs;
  // Every stage but a K tail, and for B every stage of a tile whose columns all lie below N, puts
  // the stage's offset in soffset (an SGPR) and keeps the lane offsets fixed: the load phase then
  // runs no VALU for its DMA, VALU that the other wave of the SIMD, busy with MFMAs, would hold
  // back.  Those loads read inside A and B whatever the range check does with soffset.  The K tail
  // stage and tiles at the right edge keep the whole offset in the VGPR, so the range check covers
  // every dword.  Which B form a tile uses is a compile-time flag of its loop version (b_fast), so
  // that the per-lane form's address math is not hoisted into every stage.
  const bool b_inside = n0 + BN <= N;
  auto dma_one = [&](int kt, int d, auto b_fast) {  // d: 0, 1 A; 2, 3 B
    const int s = kt % NSTAGE, i = d & 1;
    const uint32_t dst = (uint32_t)((s * STAGE_H + (wave * 2 + i) * 512) * 2);
    const bool tail = K % BK != 0 && kt == KT - 1;
    if (d < 2) {
      if (!tail) {
        eas_dma16s(ra, a_off[i], (uint32_t)(kt * BK * 2), lds_a + dst);
      } else {
        uint32_t off = a_off[i] + (uint32_t)(kt * BK * 2);
        if (kt * BK + a_k[i] >= K || a_off[i] >= 0x80000000u) off = 0x80000000u;  // past K or M: zeros
        eas_dma16(ra, off, lds_a + dst);
      }
    } else {
      if (decltype(b_fast)::value && !tail) {
        eas_dma16s(rb, b_off[i], (uint32_t)kt * (uint32_t)(BK * 2) * (uint32_t)ldb, lds_b + dst);
      } else {
        uint32_t off = b_off[i] + (uint32_t)kt * (uint32_t)(BK * 2) * (uint32_t)ldb;
        if (K % BK != 0 && kt * BK + b_k[i] >= K) off = 0x80000000u;  // B rows past K
        eas_dma16(rb, off, lds_b + dst);
      }
    }
  };
  int fa_off[2][4], fb_off[2][2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = g * 128 + i * 32 + (lane & 31);
      const int c = (2 * ks + (lane >> 5)) ^ ((r >> 2) & 3);
      fa_off[ks][i] = r * BK + c * 8;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // ds_read_b64_tr_b16: in each 16-lane group, source lane kq addresses row kq/4, columns 4(kq%4)..+3;
        // result lane i receives column i for the four rows
        const int gq = lane >> 4, kq = lane & 15;
        const int row = 16 * ks + 8 * (gq >> 1) + 4 * h + (kq >> 2);
        const int col = p * 64 + j * 32 + 16 * (gq & 1) + 4 * (kq & 3);
        const int chunk = (col >> 3) ^ bsw(row);
        fb_off[ks][j][h] = row * BN + chunk * 8 + (col & 7);
      }
  }
  // MI == 16: lane l holds A[row 16 i + l%16][k 8(l/16)..+7] and B[k 8(l/16)..+7][col 16 j + l%16]
  int fa16_off[8], fb16_off[4][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = g * 128 + i * 16 + (lane & 15);
    fa16_off[i] = r * BK + (((lane >> 4) ^ ((r >> 2) & 3)) * 8);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int gq = lane >> 4, kq = lane & 15;
      const int row = 8 * gq + 4 * h + (kq >> 2);
      const int col = p * 64 + j * 16 + 4 * (kq & 3);
      const int chunk = (col >> 3) ^ bsw(row);
      fb16_off[j][h] = row * BN + chunk * 8 + (col & 7);
    }
  eas_h8 fa[2][4], fb[2][2], fa16[8], fb16[4];
  auto read_a = [&](int s, int ks, int i) { fa[ks][i] = *(const eas_h8*)(As + s * STAGE_H + fa_off[ks][i]); };
  auto read_tr = [&](const eas_op_t* bs, int o0, int o1) {
    const eas_h4t lo = EAS_DS_TR16((EAS_LDS eas_h4t*)(bs + o0));
    const eas_h4t hi = EAS_DS_TR16((EAS_LDS eas_h4t*)(bs + o1));
    const eas_h4 l4 = __builtin_bit_cast(eas_h4, lo), h4 = __builtin_bit_cast(eas_h4, hi);
    return (eas_h8){l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
  };
  // The h = 1 half of a transposing B read is rows 4 further down with the same swizzle (rows r and
  // r + 4 differ only in bit 2, which the swizzle does not read), i.e. fb*_off[..][1] is
  // fb*_off[..][0] + 4 BN: written so, the compiler needs one address per read pair, not two.
  auto read_b = [&](int s, int ks, int j) {
    fb[ks][j] = read_tr(Bs + s * STAGE_H, fb_off[ks][j][0], fb_off[ks][j][0] + 4 * BN);
  };
  auto read_a16 = [&](int s, int i) { fa16[i] = *(const eas_h8*)(As + s * STAGE_H + fa16_off[i]); };
  auto read_b16 = [&](int s, int j) { fb16[j] = read_tr(Bs + s * STAGE_H, fb16_off[j][0], fb16_off[j][0] + 4 * BN); };
  eas_f32x16 acc[4][2];
  eas_f32x4 acc16[8][4];
  if constexpr (MI == 32) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = (eas_f32x16){};
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc16[i][j] = (eas_f32x4){};
  }
  // this wave's loads of the awaited stage are done; `later` newer stages (4 loads each) may stay in flight
  auto wait_stage = [&](int later) {
    if (later >= 2) __builtin_amdgcn_s_waitcnt(EAS_WAITVM(8));
    else if (later == 1) __builtin_amdgcn_s_waitcnt(EAS_WAITVM(4));
    else __builtin_amdgcn_s_waitcnt(EAS_WAITVM(0));
  };

  // Barrier schedule (b = workgroup barrier index): stage kt is read by group 0 between b(2kt+1)
  // and b(2kt+2) and by group 1 between b(2kt+2) and b(2kt+3).  Every wave waits for its own DMA
  // of stage kt+1 before b(2kt+2): group 0 at the end of its MFMA phase, group 1 at the end of its
  // load phase.  Stage kt+3 refills the buffer of stage kt-1, whose last reader (group 1) passed
  // b(2kt) before any wave issues that DMA.  Both groups execute the same number of barriers: group 1
  // one more before the loop, group 0 one more at the end of its last MFMA phase.
  // one stage of the K loop (s = kt % NSTAGE)
  auto stage = [&](const int kt, const int s, auto b_fast) {
    const int later = KT - 2 - kt < NSTAGE - 2 ? KT - 2 - kt : NSTAGE - 2;
    // load phase: every fragment of stage kt, and this wave's quarter of stage kt+3
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (kt + NSTAGE - 1 < KT) dma_one(kt + NSTAGE - 1, u, b_fast);
      if constexpr (MI == 32) {
        read_a(s, u >> 1, 2 * (u & 1));
        read_a(s, u >> 1, 2 * (u & 1) + 1);
        read_b(s, u >> 1, u & 1);
      } else {
        read_a16(s, 2 * u);
        read_a16(s, 2 * u + 1);
        read_b16(s, u);
      }
    }
    if (g == 1 && kt + 1 < KT) wait_stage(later);
    if constexpr (K % 8 != 0) {
      if (kt == KT - 1) {  // tail stage: halves at k >= K hold the next row of A
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (MI == 32) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
              const bool past = kt * BK + 16 * ks + 8 * (lane >> 5) + e >= K;
#pragma unroll
              for (int i = 0; i < 4; ++i) fa[ks][i][e] = past ? (eas_op_t)0.0f : fa[ks][i][e];
            }
          } else {
            const bool past = kt * BK + 8 * (lane >> 4) + e >= K;
#pragma unroll
            for (int i = 0; i < 8; ++i) fa16[i][e] = past ? (eas_op_t)0.0f : fa16[i][e];
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(EAS_WAITLGKM0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    // MFMA phase
    if constexpr (MI == 32) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = EAS_MFMA32(fa[ks][i], fb[ks][j], acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc16[i][j] = EAS_MFMA16(fa16[i], fb16[j], acc16[i][j], 0, 0, 0);
    }
    if (g == 0 && kt + 1 < KT) wait_stage(later);
    __builtin_amdgcn_sched_barrier(0);
    // group 1's barrier after its last MFMA phase would only pair with one more of group 0's:
    // both are left out (the counts stay equal), so group 0's C stores overlap that phase
    if (g == 0 || kt + 1 < KT) __syncthreads();
  };
  auto k_loop = [&](auto b_fast) {
#pragma unroll
    for (int s = 0; s < NSTAGE - 1; ++s)
      if (s < KT)
#pragma unroll
        for (int d = 0; d < 4; ++d) dma_one(s, d, b_fast);
    wait_stage(KT - 1 < NSTAGE - 2 ? KT - 1 : NSTAGE - 2);
    __syncthreads();
    if (g == 1) __syncthreads();
    for (int kt = 0; kt < KT; ++kt) stage(kt, kt % NSTAGE, b_fast);
  };
  if (b_inside)  // uniform over the workgroup
    k_loop(eas_bool_c<true>{});
  else
    k_loop(eas_bool_c<false>{});
  // the K loop is done: no LDS is read or written below
  const bool full = (m0 + BM <= M) && (n0 + BN <= N);
  if constexpr (MI == 32) {
    // lane l, register r of a 32x32 tile holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + g * 128 + i * 32 + (r / 4) * 8 + (lane >> 5) * 4 + (r % 4);
          const int col = n0 + p * 64 + j * 32 + (lane & 31);
          if (full || (row < M && col < N)) C[(size_t)row * ldb + col] = (CT)acc[i][j][r];
        }
  } else {
    // lane l, register r of a 16x16 tile holds (row 4*(l/16) + r, col l%16)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + g * 128 + i * 16 + (lane >> 4) * 4 + r;
          const int col = n0 + p * 64 + j * 16 + (lane & 15);
          if (full || (row < M && col < N)) C[(size_t)row * ldb + col] = (CT)acc16[i][j][r];
        }
  }
}

// Guard body of the 8-wave and smaller-tile entries for inputs the DMA cannot take (the launch plan
// sends those to the 4-wave entry; this path only keeps a mistaken plan correct): one f32 dot
// product per element of the TM x TN tile.
template <typename AT, typename BT, typename CT, int K, int TM = 256, int TN = TM>
static __device__ __forceinline__ void eas_gemm_elementwise(const AT* __restrict__ A, const BT* __restrict__ B,
                                                            CT* __restrict__ C, int ldb, int M, int N, int m0, int n0) {
  for (int e = threadIdx.x; e < TM * TN; e += blockDim.x) {
    const int row = m0 + e / TN, col = n0 + e % TN;
    if (row >= M || col >= N) continue;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k)
      acc = __builtin_fmaf((float)(eas_op_t)A[(size_t)row * K + k], (float)(eas_op_t)B[(size_t)k * ldb + col], acc);
    C[(size_t)row * ldb + col] = (CT)acc;
  }
}

// BM x BN tile body (128 x 64, 128 x 128, 128 x 256 or 64 x 64) for launches whose 256 x 256 grid
// would leave CUs idle: 8 waves (512 threads), specialised like the fp32 entries, on a ring of 4
// stages of BM / 16 KB of A and BN / 16 KB of B.  Waves 4-7 produce: the DMA of stage kt+3,
// BM / 64 A + BN / 64 B loads of 1 KB per wave per stage, with the stage offset in soffset, so the
// loads cost the MFMA waves sharing their SIMDs nothing.  Waves 0-3 consume, BM/2 x BN/2 each
// (MI 16: BM/32 x BN/32 accumulators of 16x16x32; MI 32: 2 x BN/64 of 32x32x16): the fragments of
// stage kt+1 are read between stage kt's MFMAs.  A load costs the SIMD that issues it tens of clocks of MFMA issue, which in a
// 4-wave form of this body (each wave loading its quarter of every stage beside its MFMAs) was
// most of the stage.
template <typename CT, int K, int BN, int MI = 16, int BM = 128>
static __device__ __forceinline__ void eas_gemm_t128(const eas_op_t* __restrict__ A, const eas_op_t* __restrict__ B,
                                                     CT* __restrict__ C, int ldb, int M, int N, int m0, int n0,
                                                     eas_op_t* smem) {
  static_assert((BN == 64 || BN == 128 || BN == 256) && (MI == 32 || MI == 16) && (BN != 64 || MI == 16) &&
                    (BM == 128 || (BM == 64 && BN == 64)),
                "128 x 64, 128 x 128, 128 x 256 or 64 x 64 tiles; 32- or 16-row MFMAs (16 on 64 columns)");
  constexpr int BK = 32, NSTAGE = 4, KT = (K + BK - 1) / BK;
  constexpr int NAI = BM / 64;              // A loads per producer wave per stage (1 or 2)
  constexpr int NJ = BN / 64;               // 32-column accumulators per consumer wave
  constexpr int NBI = BN / 64;              // B loads per producer wave per stage (1, 2 or 4)
  constexpr int CH = BN / 8;                // 16-byte chunks per B row
  constexpr int STAGE_A = BM * BK, STAGE_B = BK * BN;  // halves per stage
  constexpr int KLAST = K - (KT - 1) * BK;  // k extent of the last stage
  eas_op_t* As = smem;
  eas_op_t* Bs = smem + NSTAGE * STAGE_A;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // B's 16-byte chunk of row r is stored at chunk ^ bsw(r).  Rows of 256 or 512 bytes: bits 2-3
  // spread the four rows of a transposing read over the banks, bit 1 keeps rows 8 apart (the two
  // 16-lane groups of a half-wave in the 16 x 16 x 32 mapping) apart.  Rows of 128 bytes (two a
  // bank cycle): 2((r/2)%2) + 4((r/8)%2), as the skinny path's.  In both, rows r and r + 4 of a
  // transposing read pair (r % 8 < 4) share the mask.
  auto bsw = [](int r) {
    return BN == 64 ? 2 * ((r >> 1) & 1) + 4 * ((r >> 3) & 1) : (4 * (r & 3)) ^ (2 * ((r >> 3) & 1));
  };
  if (wave >= 4) {
    // DMA instructions write 1 KB of a stage each.  A instruction q = 2 pw + i: rows 16q + lane/4,
    // chunk lane%4 stored at chunk ^ ((row/4)%4).  B instruction q = NBI pw + i: rows
    // (64 / CH) q + lane / CH, chunk lane % CH stored at chunk ^ bsw(row).
    // Rows past M load zeros, and so do columns past N when no 8-column chunk straddles N, so
    // every address a load reads, lane offset plus stage offset, lies inside A or B.  An edge tile
    // whose chunk straddles N (N % 8 != 0) adds the stage offset to the lane offset instead, where
    // the range check sees all of it.  The last stage of a K that is not a multiple of BK does the
    // same (its straddling A chunk may end past A); stages past K load zeros into a slot nobody
    // reads, so every stage issues the same loads and the count at each barrier is the same.
    const int pw = wave - 4;
    const eas_rsrc ra = eas_make_rsrc(A, (uint32_t)M * (uint32_t)K * 2u);
    const eas_rsrc rb = eas_make_rsrc(B, ((uint32_t)(K - 1) * (uint32_t)ldb + (uint32_t)N) * 2u);
    const uint32_t lds_a = (uint32_t)(size_t)(EAS_LDS eas_op_t*)As, lds_b = (uint32_t)(size_t)(EAS_LDS eas_op_t*)Bs;
    uint32_t a_off[NAI], a_tail[NAI], b_raw[NBI], b_off[NBI], b_tail[NBI];
#pragma unroll
    for (int i = 0; i < NAI; ++i) {
      const int q = pw * NAI + i;
      const int r_a = 16 * q + (lane >> 2);
      const int c_a = (lane & 3) ^ ((r_a >> 2) & 3);
      const uint32_t a_raw = ((uint32_t)(m0 + r_a) * (uint32_t)K + (uint32_t)(c_a * 8)) * 2u;
      a_off[i] = m0 + r_a < M ? a_raw : 0x80000000u;
      a_tail[i] = (m0 + r_a < M && c_a * 8 < KLAST) ? a_raw + (uint32_t)((KT - 1) * BK * 2) : 0x80000000u;
    }
#pragma unroll
    for (int i = 0; i < NBI; ++i) {
      const int q = pw * NBI + i;
      const int r_b = (64 / CH) * q + lane / CH;
      const int c_b = (lane % CH) ^ bsw(r_b);
      b_raw[i] = ((uint32_t)r_b * (uint32_t)ldb + (uint32_t)(n0 + c_b * 8)) * 2u;
      b_off[i] = n0 + c_b * 8 < N ? b_raw[i] : 0x80000000u;
      b_tail[i] = r_b < KLAST ? b_raw[i] + (uint32_t)((KT - 1) * BK * 2) * (uint32_t)ldb : 0x80000000u;
    }
    auto dma = [&](int kt, auto b_fast) {
      const uint32_t st_a = lds_a + (uint32_t)((kt % NSTAGE) * STAGE_A * 2);
      const uint32_t st_b = lds_b + (uint32_t)((kt % NSTAGE) * STAGE_B * 2);
      const uint32_t sa = (uint32_t)(kt * BK * 2), sb = (uint32_t)(kt * BK * 2) * (uint32_t)ldb;
#pragma unroll
      for (int i = 0; i < NAI; ++i) {
        const uint32_t dst = st_a + (uint32_t)((pw * NAI + i) * 1024);
        if (kt >= KT)
          eas_dma16s(ra, 0x80000000u, 0u, dst);
        else if (K % BK != 0 && kt == KT - 1)
          eas_dma16s(ra, a_tail[i], 0u, dst);
        else
          eas_dma16s(ra, a_off[i], sa, dst);
      }
#pragma unroll
      for (int i = 0; i < NBI; ++i) {
        const uint32_t dst = st_b + (uint32_t)((pw * NBI + i) * 1024);
        if (kt >= KT)
          eas_dma16s(rb, 0x80000000u, 0u, dst);
        else if (K % BK != 0 && kt == KT - 1)
          eas_dma16s(rb, b_tail[i], 0u, dst);
        else if constexpr (decltype(b_fast)::value)
          eas_dma16s(rb, b_off[i], sb, dst);
        else
          eas_dma16s(rb, b_raw[i] + sb, 0u, dst);
      }
    };
    // one barrier per stage, as many as the consumers
    auto produce = [&](auto b_fast) {
      constexpr int PER = NAI + NBI;  // loads per stage
#pragma unroll
      for (int p = 0; p < NSTAGE - 1; ++p) dma(p, b_fast);
      __builtin_amdgcn_s_waitcnt(EAS_WAITVM(2 * PER));  // stage 0 landed (stages 1 and 2 may be in flight)
      __syncthreads();
      for (int kt = 0; kt + 1 < KT; ++kt) {
        __builtin_amdgcn_s_waitcnt(EAS_WAITVM(PER));  // stage kt+1 landed (stage kt+2 may be in flight)
        __syncthreads();
        dma(kt + NSTAGE - 1, b_fast);  // the slot of stage kt-1, whose fragments every consumer has read
      }
      __builtin_amdgcn_s_waitcnt(EAS_WAITVM(0));
    };
    if (n0 + BN <= N || N % 8 == 0)
      produce(eas_bool_c<true>{});
    else
      produce(eas_bool_c<false>{});
    return;
  }
  const int wm = wave >> 1, wn = wave & 1;
  // Fragments per stage: 4 of A and BN / 32 of B, 8 halves a lane each.  MI 32
  // (v_mfma_f32_32x32x16): A f = 2 ks + i holds A[row 32 i + l%32][k 16 ks + 8(l/32)..+7], B f =
  // ks NJ + j holds B[k 16 ks + 8(l/32)..+7][col 32 j + l%32]; MI 16 (v_mfma_f32_16x16x32): A f = i
  // holds A[row 16 i + l%16][k 8(l/16)..+7], B f = j holds B[k 8(l/16)..+7][col 16 j + l%16]
  // (rows and columns within the wave's 64 x BN/2).
  constexpr int NA = MI == 32 ? 4 : BM / 32, NB = BN / 32;  // MI 16: BM / 32 row tiles of 16 per wave
  int fa_off[NA], fb_off[NB];
#pragma unroll
  for (int f = 0; f < NA; ++f) {
    const int r = MI == 32 ? wm * 64 + (f & 1) * 32 + (lane & 31) : wm * (BM / 2) + f * 16 + (lane & 15);
    const int c = MI == 32 ? (2 * (f >> 1) + (lane >> 5)) : (lane >> 4);
    fa_off[f] = r * BK + ((c ^ ((r >> 2) & 3)) * 8);
  }
#pragma unroll
  for (int f = 0; f < NB; ++f) {
    // ds_read_b64_tr_b16: in each 16-lane group, source lane kq addresses row kq/4, columns
    // 4(kq%4)..+3; the second read of a pair (rows 4 further down) is 4 BN halves on
    const int gq = lane >> 4, kq = lane & 15;
    const int row = MI == 32 ? 16 * (f / NJ) + 8 * (gq >> 1) + (kq >> 2) : 8 * gq + (kq >> 2);
    const int col = MI == 32 ? wn * (BN / 2) + (f % NJ) * 32 + 16 * (gq & 1) + 4 * (kq & 3)
                             : wn * (BN / 2) + f * 16 + 4 * (kq & 3);
    fb_off[f] = row * BN + ((col >> 3) ^ bsw(row)) * 8 + (col & 7);
  }
  eas_f32x16 acc[2][NJ];      // MI 32: [i][j] tiles of 32 x 32
  eas_f32x4 acc16[NA][NB];    // MI 16: [i][j] tiles of 16 x 16
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = (eas_f32x16){};
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc16[i][j] = (eas_f32x4){};
  typedef eas_h8 afrag_t[NA];
  typedef eas_h8 bfrag_t[NB];
  auto read_stage = [&](int kt, afrag_t& fa, bfrag_t& fb) {
    const eas_op_t* as = As + (kt % NSTAGE) * STAGE_A;
    const eas_op_t* bs = Bs + (kt % NSTAGE) * STAGE_B;
#pragma unroll
    for (int f = 0; f < NA; ++f) fa[f] = *(const eas_h8*)(as + fa_off[f]);
#pragma unroll
    for (int f = 0; f < NB; ++f) {
      const eas_h4t lo = EAS_DS_TR16((EAS_LDS eas_h4t*)(bs + fb_off[f]));
      const eas_h4t hi = EAS_DS_TR16((EAS_LDS eas_h4t*)(bs + fb_off[f] + 4 * BN));
      const eas_h4 l4 = __builtin_bit_cast(eas_h4, lo), h4 = __builtin_bit_cast(eas_h4, hi);
      fb[f] = (eas_h8){l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
    }
  };
  auto mfmas = [&](const afrag_t& fa, const bfrag_t& fb) {
    if constexpr (MI == 32) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j) acc[i][j] = EAS_MFMA32(fa[2 * ks + i], fb[ks * NJ + j], acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < NA; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc16[i][j] = EAS_MFMA16(fa[i], fb[j], acc16[i][j], 0, 0, 0);
    }
  };
  // At the barrier of stage kt the producers' DMA of stage kt+1 has landed; after it the wave
  // issues stage kt's MFMAs from the fragments read one stage earlier and, between them, every
  // fragment read of stage kt+1 into the other set.  After this barrier the producers refill the
  // slot of stage kt-1, whose fragments every consumer read (and used) before it.
  auto step = [&](int kt, const afrag_t& fa, const bfrag_t& fb, afrag_t& na, bfrag_t& nb) {
    constexpr int NMFMA = MI == 32 ? 4 * NJ : NA * NB, NREAD = NA + 2 * NB;
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_stage(kt + 1, na, nb);
    mfmas(fa, fb);
#pragma unroll
    for (int s = 0; s < NREAD / 2; ++s) {  // the LDS reads two by two after the first MFMAs
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NMFMA - NREAD / 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // the last stage of a K that is not a multiple of 8: halves at k >= K hold the next row of A
  auto mask_tail = [&](afrag_t& fa) {
    if constexpr (K % 8 != 0) {
#pragma unroll
      for (int f = 0; f < NA; ++f)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = (KT - 1) * BK + (MI == 32 ? 16 * (f >> 1) + 8 * (lane >> 5) : 8 * (lane >> 4)) + e;
          fa[f][e] = k >= K ? (eas_op_t)0.0f : fa[f][e];
        }
    }
  };
  __syncthreads();  // stage 0 landed
  afrag_t a0, a1;
  bfrag_t b0, b1;
  read_stage(0, a0, b0);
  int kt = 0;
  for (; kt + 2 < KT; kt += 2) {  // two stages per iteration: the fragment sets alternate
    step(kt, a0, b0, a1, b1);
    step(kt + 1, a1, b1, a0, b0);
  }
  if constexpr (KT % 2 == 0) {
    step(KT - 2, a0, b0, a1, b1);
    mask_tail(a1);
    mfmas(a1, b1);
  } else {
    mask_tail(a0);
    mfmas(a0, b0);
  }
  const bool full = (m0 + BM <= M) && (n0 + BN <= N);
  if constexpr (MI == 32) {
    // lane l, register r of a 32x32 tile holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm * 64 + i * 32 + (r / 4) * 8 + (lane >> 5) * 4 + (r % 4);
          const int col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
          if (full || (row < M && col < N)) C[(size_t)row * ldb + col] = (CT)acc[i][j][r];
        }
  } else {
    // lane l, register r of a 16x16 tile holds (row 4*(l/16) + r, col l%16)
#pragma unroll
    for (int i = 0; i < NA; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + wm * (BM / 2) + i * 16 + (lane >> 4) * 4 + r;
          const int col = n0 + wn * (BN / 2) + j * 16 + (lane & 15);
          if (full || (row < M && col < N)) C[(size_t)row * ldb + col] = (CT)acc16[i][j][r];
        }
  }
}

// Skinny path (M <= 128, decode-like): one workgroup per NT = 64 columns (128 for launches whose
// 64-column groups would need more than one round of CUs), the four waves split K.  Each wave
// streams its K range of B (and A) HBM -> LDS into a private ring of 4 stages (3 or 2 where 4
// would not fit the LDS; no barriers in the loop), multiplies MT row tiles of 16
// (1, 2, 4 or 8) by NT / 16 column tiles with v_mfma_f32_16x16x32_f16 (B transposed by
// ds_read_b64_tr_b16), and the waves add their 16 MT x NT partial sums through LDS at the end.
template <typename CT, int K, int MT, int NT = 64>
static __device__ __forceinline__ void eas_gemm_skinny_dma(const eas_op_t* __restrict__ A, const eas_op_t* __restrict__ B,
                                                           CT* __restrict__ C, int ldb, int M, int N, int n0,
                                                           eas_op_t* smem) {
  static_assert(NT == 64 || NT == 128, "64 or 128 columns per workgroup");
  typedef float eas_f32x4_acc __attribute__((ext_vector_type(4)));
  constexpr int KS = 32, MR = 16 * MT, NJ = NT / 16;
  constexpr int KW = ((K + 4 * KS - 1) / (4 * KS)) * KS;  // k rows per wave
  constexpr int BST = KS * NT, AST = MR * KS, STH = BST + AST;  // halves per stage: B [32][NT], A [MR][32]
  constexpr int NST = 4 * 4 * STH * 2 <= 147456 ? 4 : 4 * 3 * STH * 2 <= 147456 ? 3 : 2;  // per wave (144 KB)
  static_assert(4 * NST * STH * 2 <= 147456, "the rings fit the entry's LDS");
  constexpr int NBQ = NT / 16, CH = NT / 8;                     // B DMA instructions per stage, chunks per row
  constexpr int LOADS = NBQ + MT;                               // DMA instructions per stage
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kb = wave * KW, ke = min(K, kb + KW);
  const int nsteps = ke > kb ? (ke - kb + KS - 1) / KS : 0;
  eas_op_t* ws = smem + wave * NST * STH;
  const uint32_t lds_ws = (uint32_t)(size_t)(EAS_LDS eas_op_t*)ws;
  const eas_rsrc ra = eas_make_rsrc(A, (uint32_t)M * (uint32_t)K * 2u);
  const eas_rsrc rb = eas_make_rsrc(B, ((uint32_t)(K - 1) * (uint32_t)ldb + (uint32_t)N) * 2u);
  // B DMA q: rows (64 / CH) q + lane / CH of the stage, chunk lane % CH stored at chunk ^ s(row).
  // 128-byte rows (NT 64): s(r) = 2((r/2)%2) + 4((r/8)%2); 256-byte rows (NT 128): s(r) =
  // 2(r%4) + 8((r/8)%2).  Either keeps each half-wave of a transposed read conflict free.
  auto swz = [](int r) { return NT == 64 ? 2 * ((r >> 1) & 1) + 4 * ((r >> 3) & 1) : 2 * (r & 3) + 8 * ((r >> 3) & 1); };
  uint32_t b_off[NBQ];
  int b_row[NBQ];
#pragma unroll
  for (int q = 0; q < NBQ; ++q) {
    const int r = (64 / CH) * q + lane / CH;
    const int lc = (lane % CH) ^ swz(r);
    b_row[q] = r;
    b_off[q] = ((uint32_t)r * (uint32_t)ldb + (uint32_t)(n0 + lc * 8)) * 2u;
  }
  // A DMA t (one per row tile): row 16t + lane/4, chunk lane%4 stored at chunk ^ ((row/4)%4)
  const int a_m = lane >> 2, a_lc = (lane & 3) ^ ((a_m >> 2) & 3);
  const uint32_t a_off = ((uint32_t)a_m * (uint32_t)K + (uint32_t)(a_lc * 8)) * 2u;
  auto dma_step = [&](int t) {
    const int k0 = kb + t * KS;
    const uint32_t dst = lds_ws + (uint32_t)((t % NST) * STH) * 2u;
#pragma unroll
    for (int q = 0; q < NBQ; ++q) {
      uint32_t off = b_off[q] + (uint32_t)k0 * (uint32_t)ldb * 2u;
      if (k0 + b_row[q] >= ke) off = 0x80000000u;  // another wave's rows, or past K: zeros
      eas_dma16(rb, off, dst + q * 1024);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      uint32_t off = a_off + ((uint32_t)(16 * mt) * (uint32_t)K + (uint32_t)k0) * 2u;
      if (k0 + a_lc * 8 >= ke) off = 0x80000000u;
      eas_dma16(ra, off, dst + BST * 2 + mt * 1024);
    }
  };
  // 16x16x32 operands: A lane l holds A[l%16][8(l/16)..+7]; B lane l holds B[8(l/16)..+7][l%16]
  const int fm = lane & 15;
  const int fa = fm * KS + (((lane >> 4) ^ ((fm >> 2) & 3)) * 8);
  int fb[NJ][2];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int g = lane >> 4, kq = lane & 15;
      const int row = 8 * g + 4 * h + (kq >> 2), col = 16 * j + 4 * (kq & 3);
      const int pc = (col >> 3) ^ swz(row);
      fb[j][h] = row * NT + pc * 8 + (col & 7);
    }
  eas_f32x4_acc acc[MT][NJ];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[mt][j] = (eas_f32x4_acc){};
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    if (p < nsteps) dma_step(p);
  for (int t = 0; t < nsteps; ++t) {
    // this wave's step t landed; up to NST-2 newer steps (LOADS loads each) stay in flight
    const int later = min(NST - 2, nsteps - 1 - t);
    if (later >= 2) __builtin_amdgcn_s_waitcnt(EAS_WAITVM(2 * LOADS));
    else if (later == 1) __builtin_amdgcn_s_waitcnt(EAS_WAITVM(LOADS));
    else __builtin_amdgcn_s_waitcnt(EAS_WAITVM(0));
    if (t + NST - 1 < nsteps) dma_step(t + NST - 1);  // refills the stage read at step t-1
    const eas_op_t* st = ws + (t % NST) * STH;
    eas_h8 a[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) a[mt] = *(const eas_h8*)(st + BST + mt * 16 * KS + fa);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const eas_h4t lo = EAS_DS_TR16((EAS_LDS eas_h4t*)(st + fb[j][0]));
      const eas_h4t hi = EAS_DS_TR16((EAS_LDS eas_h4t*)(st + fb[j][1]));
      const eas_h4 l4 = __builtin_bit_cast(eas_h4, lo), h4 = __builtin_bit_cast(eas_h4, hi);
      const eas_h8 b = (eas_h8){l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt][j] = EAS_MFMA16(a[mt], b, acc[mt][j], 0, 0, 0);
    }
  }
  // The waves' partial sums meet in LDS, RP rows at a time: [4 waves][RP][NT] floats must fit the
  // entry's 144 KB (all rows at once, except 8 row tiles on 128 columns: two passes of 64 rows).
  constexpr int RP = 4 * MR * NT * 4 <= 147456 ? MR : 64;
  static_assert(4 * RP * NT * 4 <= 147456 && MR % RP == 0, "the reduction fits the LDS");
  float* red = (float*)smem;  // [4 waves][RP][NT]
#pragma unroll
  for (int p0 = 0; p0 < MR; p0 += RP) {
    __syncthreads();  // every wave is past its K loop (first pass) or the previous pass's reads
    // 16x16 D layout: lane l, register r holds (row 4(l/16) + r, col l%16)
#pragma unroll
    for (int mt = p0 / 16; mt < (p0 + RP) / 16; ++mt)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[(wave * RP + 16 * mt - p0 + 4 * (lane >> 4) + r) * NT + 16 * j + (lane & 15)] = acc[mt][j][r];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < RP * NT / 256; ++e) {
      const int idx = tid + 256 * e, row = idx / NT, col = idx % NT;
      const float sum = (red[row * NT + col] + red[(RP + row) * NT + col]) +
                        (red[(2 * RP + row) * NT + col] + red[(3 * RP + row) * NT + col]);
      if (p0 + row < M && n0 + col < N) C[(size_t)(p0 + row) * ldb + n0 + col] = (CT)sum;
    }
  }
}

// Skinny path for inputs the DMA cannot take (f32 or unaligned): one thread per (column, 4 MT rows)
// of the 64 columns from n0.
template <typename AT, typename BT, typename CT, int K, int MT>
static __device__ __forceinline__ void eas_gemm_skinny_simple(const AT* __restrict__ A, const BT* __restrict__ B,
                                                              CT* __restrict__ C, int ldb, int M, int N, int n0) {
  constexpr int R = 4 * MT;  // rows per thread: r0, r0 + 4, ...
  const int tid = threadIdx.x, col = n0 + (tid & 63), r0 = tid >> 6;
  if (col >= N) return;
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = 0.0f;
  for (int k = 0; k < K; ++k) {
    const float b = (float)(eas_op_t)B[(size_t)k * ldb + col];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = r0 + 4 * i;
      const float a = row < M ? (float)(eas_op_t)A[(size_t)row * K + k] : 0.0f;
      acc[i] = __builtin_fmaf(a, b, acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (r0 + 4 * i < M) C[(size_t)(r0 + 4 * i) * ldb + col] = (CT)acc[i];
}

template <typename AT, typename BT, typename CT, int K>
static __device__ __forceinline__ void eas_gemm_regs(const AT* __restrict__ A, const BT* __restrict__ B,
                                                     CT* __restrict__ C, int ldb, int M, int N, int m0, int n0,
                                                     eas_op_t* smem) {
  constexpr int BM = 256, BN = 256, BK = 64, WN = 2, NTHREADS = 256, TI = 4, TJ = 4;
  constexpr int PITCH = BK + 8, KC = BK / 8, A_IT = BM * BK / 8 / NTHREADS, NBLK = BK * BN / 64;
  constexpr int B_IT = (NBLK + NTHREADS - 1) / NTHREADS;
  eas_op_t* As0 = smem;  // [2][BM * PITCH]
  eas_op_t* Bs0 = smem + 2 * BM * PITCH;  // [2][BN * PITCH]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  // A rows (length K, compile time) load A_AL elements per vector; B rows need 16-byte vectors
  // (ldb a multiple of 16 bytes, aligned base).  Anything else takes the masked element path.
  constexpr int A_AL = eas_row_vec<AT>(K);
  const bool mn_full = (m0 + BM <= M) && (n0 + BN <= N) && (ldb % (16 / (int)sizeof(BT)) == 0) &&
                       ((uint64_t)B % 16 == 0) && ((uint64_t)A % (A_AL * sizeof(AT)) == 0);

  eas_h8 ra[A_IT], rb[B_IT][8];
  auto gload_fast = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + NTHREADS * i, row = c / KC, kc = c % KC;
      ra[i] = eas_load8_al<AT, A_AL>(A + (size_t)(m0 + row) * K + k0 + kc * 8);
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int blk = tid + NTHREADS * i, kg = blk % KC, nc = blk / KC;
      if (NBLK % NTHREADS != 0 && blk >= NBLK) break;
#pragma unroll
      for (int r = 0; r < 8; ++r) rb[i][r] = eas_load8<BT>(B + (size_t)(k0 + kg * 8 + r) * ldb + n0 + nc * 8);
    }
  };
  auto sstore_regs = [&](int buf) {
    eas_op_t* As = As0 + buf * BM * PITCH;
    eas_op_t* Bs = Bs0 + buf * BN * PITCH;
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + NTHREADS * i, row = c / KC, kc = c % KC;
      *(eas_h8*)(&As[row * PITCH + kc * 8]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int blk = tid + NTHREADS * i, kg = blk % KC, nc = blk / KC;
      if (NBLK % NTHREADS != 0 && blk >= NBLK) break;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        eas_h8 col;
#pragma unroll
        for (int r = 0; r < 8; ++r) col[r] = rb[i][r][j];
        *(eas_h8*)(&Bs[(nc * 8 + j) * PITCH + kg * 8]) = col;
      }
    }
  };
  // edge tiles and the K tail: element loads with zero fill, written straight to LDS
  // (rolled loops keep register pressure low; these tiles are few)
  auto sstore_masked = [&](int buf, int k0) {
    eas_op_t* As = As0 + buf * BM * PITCH;
    eas_op_t* Bs = Bs0 + buf * BN * PITCH;
#pragma unroll 1
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + NTHREADS * i, row = c / KC, kc = c % KC;
      const int gm_ = m0 + row, gk = k0 + kc * 8;
      eas_h8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (gm_ < M && gk + e < K) ? (eas_op_t)A[(size_t)gm_ * K + gk + e] : (eas_op_t)0.0f;
      *(eas_h8*)(&As[row * PITCH + kc * 8]) = v;
    }
#pragma unroll 1
    for (int i = 0; i < B_IT; ++i) {
      const int blk = tid + NTHREADS * i, kg = blk % KC, nc = blk / KC;
      if (NBLK % NTHREADS != 0 && blk >= NBLK) break;
      const int gn = n0 + nc * 8;
#pragma unroll 1
      for (int j = 0; j < 8; ++j) {
        eas_h8 col;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int gk = k0 + kg * 8 + r;
          col[r] = (gk < K && gn + j < N) ? (eas_op_t)B[(size_t)gk * ldb + gn + j] : (eas_op_t)0.0f;
        }
        *(eas_h8*)(&Bs[(nc * 8 + j) * PITCH + kg * 8]) = col;
      }
    }
  };
  eas_f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = (eas_f32x16){};

  constexpr int KT = (K + BK - 1) / BK, KFULL = K / BK;
  auto compute = [&](int kt) {
    const eas_op_t* As = As0 + (kt & 1) * BM * PITCH;
    const eas_op_t* Bs = Bs0 + (kt & 1) * BN * PITCH;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      eas_h8 a[TI], b[TJ];
      const int kk = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TI; ++i) a[i] = *(const eas_h8*)&As[(wm * 128 + i * 32 + (lane & 31)) * PITCH + kk];
#pragma unroll
      for (int j = 0; j < TJ; ++j) b[j] = *(const eas_h8*)&Bs[(wn * 128 + j * 32 + (lane & 31)) * PITCH + kk];
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = EAS_MFMA32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };
  if (mn_full) {
    // interior tile: full k-tiles stage through registers, loads issued before the current MFMAs
    if (KFULL > 0) {
      gload_fast(0);
      sstore_regs(0);
    } else {
      sstore_masked(0, 0);
    }
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      const bool next_fast = kt + 1 < KFULL;
      if (next_fast) gload_fast((kt + 1) * BK);
      compute(kt);
      if (next_fast) sstore_regs((kt + 1) & 1);
      else if (kt + 1 < KT) sstore_masked((kt + 1) & 1, (kt + 1) * BK);  // the K tail
      __syncthreads();
    }
  } else {
    sstore_masked(0, 0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      compute(kt);
      if (kt + 1 < KT) sstore_masked((kt + 1) & 1, (kt + 1) * BK);
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 128 + i * 32 + (r / 4) * 8 + (lane >> 5) * 4 + (r % 4);
        const int col = n0 + wn * 128 + j * 32 + (lane & 31);
        if (mn_full || (row < M && col < N)) C[(size_t)row * ldb + col] = (CT)acc[i][j][r];
      }
}

// Origin of this workgroup's BM x BN tile: XCD-contiguous (workgroup w runs on XCD w % 8, so
// each XCD gets a contiguous range of tiles), grouped 4 tile-rows high for L2 reuse.
template <int BM = 256, int BN = 256>
static __device__ __forceinline__ void eas_tile_origin(int M, int N, int& m0, int& n0) {
  constexpr int GROUP_M = 4;
  const int tilesM = (M + BM - 1) / BM, tilesN = (N + BN - 1) / BN, T = tilesM * tilesN;
  const int w = blockIdx.x;
  const int t = (T % 8 == 0) ? (w % 8) * (T / 8) + w / 8 : w;
  const int gsize = GROUP_M * tilesN, g = t / gsize, first_m = g * GROUP_M;
  const int gm = min(tilesM - first_m, GROUP_M);
  m0 = (first_m + (t % gsize) % gm) * BM;
  n0 = ((t % gsize) / gm) * BN;
}

extern "C" __global__ __launch_bounds__(256) void @NAME@(
    @PARAMS@) {
  constexpr int K = @K@, SKINNY_M = @SKINNY_M@;
  constexpr bool OP_IN = @OP_IN@;
  typedef @AT@ AT;
  typedef @BT@ BT;
  typedef @CT@ CT;
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const AT* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const BT* __restrict__ B = @B@ + __eas_n_lo;
  CT* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  // one LDS array for all bodies: DMA ring 4 x 2 x 16 KB, register body 2 x 2 x 256 x 72 halves,
  // skinny path 4 waves x 4 stages x (4 + MT) KB (3 stages x 12 KB for 8 row tiles)
  __shared__ __attribute__((aligned(1024))) eas_op_t smem[2 * 2 * 256 * 72];
  // DMA loads take any 4-byte aligned rows (16-byte chunks may straddle alignment and the buffer range,
  // which is checked per dword); the skinny path also wants whole 16-byte chunks per row of A
  const bool dma_ok = OP_IN && (K % 2 == 0) && (ldb % 2 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 4 == 0) &&
                      ((uint64_t)M * K * 2 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 2 < (1ull << 31));
  const bool skinny_dma_ok = dma_ok && (K % 8 == 0) && (ldb % 8 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 16 == 0);
  if (M <= SKINNY_M) {
    // The launch plan gives one workgroup per 64 columns, or per 128 when that keeps the launch to
    // one round of CUs; the grid says which.  1, 2, 4 or 8 row tiles of 16.
    const bool wide = (int)gridDim.x * 64 < N;
    const int n0 = (int)blockIdx.x * (wide ? 128 : 64);
    if constexpr (OP_IN) {
      if (skinny_dma_ok) {
        const eas_op_t* __restrict__ Ah = (const eas_op_t*)A;
        const eas_op_t* __restrict__ Bh = (const eas_op_t*)B;
        if (wide) {
          if (M <= 16) eas_gemm_skinny_dma<CT, K, 1, 128>(Ah, Bh, C, ldb, M, N, n0, smem);
          else if (M <= 32) eas_gemm_skinny_dma<CT, K, 2, 128>(Ah, Bh, C, ldb, M, N, n0, smem);
          else if (M <= 64) eas_gemm_skinny_dma<CT, K, 4, 128>(Ah, Bh, C, ldb, M, N, n0, smem);
          else eas_gemm_skinny_dma<CT, K, 8, 128>(Ah, Bh, C, ldb, M, N, n0, smem);
          return;
        } else {
          if (M <= 16) eas_gemm_skinny_dma<CT, K, 1>(Ah, Bh, C, ldb, M, N, n0, smem);
          else if (M <= 32) eas_gemm_skinny_dma<CT, K, 2>(Ah, Bh, C, ldb, M, N, n0, smem);
          else if (M <= 64) eas_gemm_skinny_dma<CT, K, 4>(Ah, Bh, C, ldb, M, N, n0, smem);
          else eas_gemm_skinny_dma<CT, K, 8>(Ah, Bh, C, ldb, M, N, n0, smem);
          return;
        }
      }
    }
    // inputs the DMA cannot take (on a 128-column grid, 64 columns at a time)
    if (M <= 16) {
      eas_gemm_skinny_simple<AT, BT, CT, K, 1>(A, B, C, ldb, M, N, n0);
      if (wide) eas_gemm_skinny_simple<AT, BT, CT, K, 1>(A, B, C, ldb, M, N, n0 + 64);
    } else if (M <= 64) {
      eas_gemm_skinny_simple<AT, BT, CT, K, 4>(A, B, C, ldb, M, N, n0);
      if (wide) eas_gemm_skinny_simple<AT, BT, CT, K, 4>(A, B, C, ldb, M, N, n0 + 64);
    } else {
      eas_gemm_skinny_simple<AT, BT, CT, K, 8>(A, B, C, ldb, M, N, n0);
      if (wide) eas_gemm_skinny_simple<AT, BT, CT, K, 8>(A, B, C, ldb, M, N, n0 + 64);
    }
    return;
  }
  int m0, n0;
  eas_tile_origin(M, N, m0, n0);
  if constexpr (OP_IN) {
    if (dma_ok) {
      eas_gemm_dma<CT, K>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);
      return;
    }
  }
  eas_gemm_regs<AT, BT, CT, K>(A, B, C, ldb, M, N, m0, n0, smem);
}
"""

# The 8-wave entry and the 128 x 128 tile entry (f16 A and B): the launch plan picks one for
# launches above the skinny height whose operands the DMA can take (the 128-tile one when the
# 256 x 256 grid would leave CUs idle).
_TEMPLATE_PP_ENTRY = r"""
extern "C" __global__ __launch_bounds__(512) void @NAME@__pp(
    @PARAMS@) {
  constexpr int K = @K@;
  typedef @AT@ AT;
  typedef @BT@ BT;
  typedef @CT@ CT;
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const AT* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const BT* __restrict__ B = @B@ + __eas_n_lo;
  CT* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  __shared__ __attribute__((aligned(1024))) eas_op_t smem[2 * 4 * 256 * 32];  // DMA ring 4 x 2 x 16 KB
  const bool dma_ok = (K % 2 == 0) && (ldb % 2 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 4 == 0) &&
                      ((uint64_t)M * K * 2 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 2 < (1ull << 31));
  int m0, n0;
  eas_tile_origin(M, N, m0, n0);
  if (dma_ok)
    eas_gemm_pp<CT, K, @PP_MI@>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);
  else
    eas_gemm_elementwise<AT, BT, CT, K>(A, B, C, ldb, M, N, m0, n0);
}

extern "C" __global__ __launch_bounds__(512) void @NAME@__t128(
    @PARAMS@) {
  constexpr int K = @K@;
  typedef @AT@ AT;
  typedef @BT@ BT;
  typedef @CT@ CT;
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const AT* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const BT* __restrict__ B = @B@ + __eas_n_lo;
  CT* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  __shared__ __attribute__((aligned(1024))) eas_op_t smem[2 * 4 * 128 * 32];  // DMA ring 4 x 2 x 8 KB
  const bool dma_ok = (K % 2 == 0) && (ldb % 2 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 4 == 0) &&
                      ((uint64_t)M * K * 2 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 2 < (1ull << 31));
  int m0, n0;
  eas_tile_origin<128, 128>(M, N, m0, n0);
  if (dma_ok)
    eas_gemm_t128<CT, K, 128, @PP_MI@>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);
  else
    eas_gemm_elementwise<AT, BT, CT, K, 128>(A, B, C, ldb, M, N, m0, n0);
}

extern "C" __global__ __launch_bounds__(512) void @NAME@__t128x256(
    @PARAMS@) {
  constexpr int K = @K@;
  typedef @AT@ AT;
  typedef @BT@ BT;
  typedef @CT@ CT;
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const AT* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const BT* __restrict__ B = @B@ + __eas_n_lo;
  CT* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  __shared__ __attribute__((aligned(1024))) eas_op_t smem[4 * (128 * 32 + 32 * 256)];  // DMA ring 4 x (8 + 16) KB
  const bool dma_ok = (K % 2 == 0) && (ldb % 2 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 4 == 0) &&
                      ((uint64_t)M * K * 2 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 2 < (1ull << 31));
  int m0, n0;
  eas_tile_origin<128, 256>(M, N, m0, n0);
  if (dma_ok)
    eas_gemm_t128<CT, K, 256, @PP_MI@>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);
  else
    eas_gemm_elementwise<AT, BT, CT, K, 128, 256>(A, B, C, ldb, M, N, m0, n0);
}

extern "C" __global__ __launch_bounds__(512) void @NAME@__t128x64(
    @PARAMS@) {
  constexpr int K = @K@;
  typedef @AT@ AT;
  typedef @BT@ BT;
  typedef @CT@ CT;
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const AT* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const BT* __restrict__ B = @B@ + __eas_n_lo;
  CT* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  __shared__ __attribute__((aligned(1024))) eas_op_t smem[4 * (128 * 32 + 32 * 64)];  // DMA ring 4 x (8 + 4) KB
  const bool dma_ok = (K % 2 == 0) && (ldb % 2 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 4 == 0) &&
                      ((uint64_t)M * K * 2 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 2 < (1ull << 31));
  int m0, n0;
  eas_tile_origin<128, 64>(M, N, m0, n0);
  if (dma_ok)
    eas_gemm_t128<CT, K, 64, 16>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);
  else
    eas_gemm_elementwise<AT, BT, CT, K, 128, 64>(A, B, C, ldb, M, N, m0, n0);
}

extern "C" __global__ __launch_bounds__(512) void @NAME@__t64x64(
    @PARAMS@) {
  constexpr int K = @K@;
  typedef @AT@ AT;
  typedef @BT@ BT;
  typedef @CT@ CT;
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const AT* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const BT* __restrict__ B = @B@ + __eas_n_lo;
  CT* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  __shared__ __attribute__((aligned(1024))) eas_op_t smem[4 * (64 * 32 + 32 * 64)];  // DMA ring 4 x (4 + 4) KB
  const bool dma_ok = (K % 2 == 0) && (ldb % 2 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 4 == 0) &&
                      ((uint64_t)M * K * 2 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 2 < (1ull << 31));
  int m0, n0;
  eas_tile_origin<64, 64>(M, N, m0, n0);
  if (dma_ok)
    eas_gemm_t128<CT, K, 64, 16, 64>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);
  else
    eas_gemm_elementwise<AT, BT, CT, K, 64, 64>(A, B, C, ldb, M, N, m0, n0);
}
"""

# The fp32 entries (the tiled threadgroup kernel lifted to v_mfma_f32_32x32x2_f32) run 8 waves
# (512 threads), specialised.  Waves 0-3 consume: fragment reads one stage ahead, interleaved one
# per MFMA with the current stage's MFMAs.  Waves 4-7 produce: the HBM -> LDS DMA of a 4-stage
# ring of BK = 32, three stages ahead, with no VALU.  Measured on MI355X, a wave that issues a
# 16-byte-per-lane load (to LDS or to VGPRs) costs its SIMD's MFMA pipe ~30 clocks, while loads
# issued by the other wave of the SIMD cost the MFMA wave nothing as long as that wave runs no
# VALU: at 1024^3 a stage of the 64 x 64 entry takes 1105 clocks instead of 1232 (1024 for its
# MFMAs), at 2048^3 one of the 128 x 128 entry 4187 instead of 4418 (4096).
_TEMPLATE_F32 = r"""
extern "C" __global__ __launch_bounds__(512) void @NAME@(
    @PARAMS@) {
  constexpr int BM = 64, BN = 64, BK = 32, NSTAGE = 4, K = @K@, KT = (K + BK - 1) / BK;
  constexpr int AST = BM * BK, BST = BK * BN, STF = AST + BST;  // floats per stage
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const float* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const float* __restrict__ B = @B@ + __eas_n_lo;
  float* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  __shared__ __attribute__((aligned(1024))) float smem[NSTAGE * STF];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-contiguous, M-grouped tile order
  const int tilesM = (M + BM - 1) / BM, tilesN = (N + BN - 1) / BN, T = tilesM * tilesN;
  const int w = blockIdx.x;
  const int t = (T % 8 == 0) ? (w % 8) * (T / 8) + w / 8 : w;
  constexpr int GROUP_M = 8;
  const int gsize = GROUP_M * tilesN, g = t / gsize, first_m = g * GROUP_M;
  const int gm = min(tilesM - first_m, GROUP_M);
  const int m0 = (first_m + (t % gsize) % gm) * BM, n0 = ((t % gsize) / gm) * BN;
  const bool dma_ok = (K % 4 == 0) && (ldb % 4 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 16 == 0) &&
                      ((uint64_t)M * K * 4 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 4 < (1ull << 31));
  if (!dma_ok) {
    // rows not 16-byte aligned: each of 256 threads accumulates a 4 x 4 block with plain fmas
    if (tid >= 256) return;
    const int r0 = m0 + (tid >> 4) * 4, c0 = n0 + (tid & 15) * 4;
    float acc[4][4] = {};
    for (int k = 0; k < K; ++k) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = r0 + i < M ? A[(size_t)(r0 + i) * K + k] : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = c0 + j < N ? B[(size_t)k * ldb + c0 + j] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (r0 + i < M && c0 + j < N) C[(size_t)(r0 + i) * ldb + c0 + j] = acc[i][j];
    return;
  }
  if (wave >= 4) {
    // producer: the DMA (1 KB per instruction, 2 A + 2 B per wave per stage, q = 2 pw + i)
    //   A stage [64 rows][32 k]: rows 8q + lane/8, 16-byte chunk lane%8 stored at chunk ^ ((row/2)%8)
    //   B stage [32 k][64 n]:    rows 4q + lane/16, chunk lane%16 stored at chunk ^ 8((row/16)%2)
    // Rows past M and columns past N load zeros (they are never stored), so every address a load
    // reads, lane offset plus stage offset, lies inside A or B.  The last stage of a K that is not
    // a multiple of BK loads zeros past K; stages past K load zeros into a slot nobody reads, so
    // every stage issues 4 loads and the count at each barrier is the same.
    const int pw = wave - 4;
    const eas_rsrc ra = eas_make_rsrc(A, (uint32_t)M * (uint32_t)K * 4u);
    const eas_rsrc rb = eas_make_rsrc(B, ((uint32_t)(K - 1) * (uint32_t)ldb + (uint32_t)N) * 4u);
    const uint32_t lds0 = (uint32_t)(size_t)(EAS_LDS float*)smem;
    constexpr int KLAST = K - (KT - 1) * BK;  // k extent of the last stage
    uint32_t a_off[2], b_off[2], a_tail[2], b_tail[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = pw * 2 + i;
      const int r = 8 * q + (lane >> 3), lc = (lane & 7) ^ ((r >> 1) & 7);
      a_off[i] = m0 + r < M ? ((uint32_t)(m0 + r) * (uint32_t)K + (uint32_t)(lc * 4)) * 4u : 0x80000000u;
      a_tail[i] = lc * 4 >= KLAST ? 0x80000000u : a_off[i];
      const int rr = 4 * q + (lane >> 4), lcb = (lane & 15) ^ (8 * ((rr >> 4) & 1));
      b_off[i] = n0 + lcb * 4 < N ? (uint32_t)(n0 + lcb * 4) * 4u + (uint32_t)rr * (uint32_t)ldb * 4u : 0x80000000u;
      b_tail[i] = rr >= KLAST ? 0x80000000u : b_off[i];
    }
    auto dma = [&](int kt) {
      const uint32_t st = lds0 + (uint32_t)((kt % NSTAGE) * STF) * 4u;
      const uint32_t sa = (uint32_t)(kt * BK) * 4u, sb = (uint32_t)(kt * BK) * (uint32_t)ldb * 4u;
      if (kt >= KT) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          eas_dma16s(ra, 0x80000000u, 0u, st + (pw * 2 + i) * 1024);
          eas_dma16s(rb, 0x80000000u, 0u, st + AST * 4 + (pw * 2 + i) * 1024);
        }
      } else if (K % BK != 0 && kt == KT - 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          eas_dma16s(ra, a_tail[i], sa, st + (pw * 2 + i) * 1024);
          eas_dma16s(rb, b_tail[i], sb, st + AST * 4 + (pw * 2 + i) * 1024);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          eas_dma16s(ra, a_off[i], sa, st + (pw * 2 + i) * 1024);
          eas_dma16s(rb, b_off[i], sb, st + AST * 4 + (pw * 2 + i) * 1024);
        }
      }
    };
    // one barrier per stage, as many as the consumers
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) dma(p);
    __builtin_amdgcn_s_waitcnt(EAS_WAITVM(8));  // stage 0 landed (stages 1 and 2 may be in flight)
    __syncthreads();
    for (int kt = 0; kt + 1 < KT; ++kt) {
      __builtin_amdgcn_s_waitcnt(EAS_WAITVM(4));  // stage kt+1 landed (stage kt+2 may be in flight)
      __syncthreads();
      dma(kt + NSTAGE - 1);  // the slot of stage kt-1, whose fragments every consumer has read
    }
    __builtin_amdgcn_s_waitcnt(EAS_WAITVM(0));
    return;
  }
  // consumers: 4 waves of 32 x 32; v_mfma_f32_32x32x2_f32: A lane l holds A[l%32][k], B lane l
  // holds B[k][l%32]
  const int wm = wave >> 1, wn = wave & 1;
  // k order within a stage: MFMA step s (0..15) takes k = s + 16 c for lane half c = lane/32, so one
  // ds_read_b128 gives a lane A values for four steps; B is one float of row s + 16 c per step
  const int c = lane >> 5, ai = wm * 32 + (lane & 31), bj = wn * 32 + (lane & 31);
  int fa[4], fb[16];
#pragma unroll
  for (int u = 0; u < 4; ++u) fa[u] = ai * BK + (((4 * c + u) ^ ((ai >> 1) & 7)) * 4);
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const int row = s + 16 * c;
    fb[s] = AST + row * BN + (((bj >> 2) ^ (8 * ((row >> 4) & 1))) * 4) + (bj & 3);
  }
  eas_f32x16 acc = {};
  // Fragments are read one stage ahead and interleaved with the MFMAs.  At the barrier of stage
  // kt the producers' DMA of stage kt+1 has landed; after it the wave issues stage kt's 16 MFMAs
  // (a dependent chain, 64 clocks each) from the register set read one stage earlier, and between
  // them the reads of stage kt+1 into the other set, one per MFMA (sched_group_barrier).  After
  // this barrier the producers refill the slot of stage kt-1, whose fragments every consumer read
  // (and waited for, at the barrier of stage kt-1) before it.
  auto read_stage = [&](int kt, eas_f32x4 (&a)[4], float (&b)[16]) {
    const float* st = smem + (kt % NSTAGE) * STF;
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = *(const eas_f32x4*)(st + fa[u]);
#pragma unroll
    for (int s = 0; s < 16; ++s) b[s] = st[fb[s]];
  };
  auto mfmas = [&](const eas_f32x4 (&a)[4], const float (&b)[16]) {
#pragma unroll
    for (int s = 0; s < 16; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s >> 2][s & 3], b[s], acc, 0, 0, 0);
  };
  // a stage that is followed by another (KT - 1 of them, each with the barrier the producers match)
  auto step = [&](int kt, const eas_f32x4 (&a)[4], const float (&b)[16], eas_f32x4 (&na)[4], float (&nb)[16]) {
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_stage(kt + 1, na, nb);
    mfmas(a, b);
    // one LDS read after each of the first 12 MFMAs
#pragma unroll
    for (int s = 0; s < 12; ++s) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  __syncthreads();  // stage 0 landed
  eas_f32x4 a0[4], a1[4];
  float b0[16], b1[16];
  read_stage(0, a0, b0);
  int kt = 0;
  for (; kt + 2 < KT; kt += 2) {  // two stages per iteration: the register sets alternate
    step(kt, a0, b0, a1, b1);
    step(kt + 1, a1, b1, a0, b0);
  }
  if constexpr (KT % 2 == 0) {
    step(KT - 2, a0, b0, a1, b1);
    mfmas(a1, b1);
  } else {
    mfmas(a0, b0);
  }
  // lane l, register r holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32)
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = m0 + wm * 32 + (r / 4) * 8 + (lane >> 5) * 4 + (r % 4);
    const int col = n0 + wn * 32 + (lane & 31);
    if (row < M && col < N) C[(size_t)row * ldb + col] = acc[r];
  }
}
"""

# The fp32 128 x 128 tile entry: four consumer waves of 64 x 64 (2 x 2 accumulators of
# v_mfma_f32_32x32x2_f32) and four producer waves, a 4-stage ring of 32 KB stages.  A quarter of
# the 64-tile kernel's DMA bytes per flop and four independent MFMA chains per wave; the launch
# plan picks it when 128 x 128 tiles still give every CU one.
_TEMPLATE_F32_T128 = r"""
extern "C" __global__ __launch_bounds__(512) void @NAME@__t128(
    @PARAMS@) {
  constexpr int BM = 128, BN = 128, BK = 32, NSTAGE = 4, K = @K@, KT = (K + BK - 1) / BK;
  constexpr int AST = BM * BK, BST = BK * BN, STF = AST + BST;  // floats per stage (32 KB)
  const int ldb = (int)@LDB@;
  // the launch rectangle [m_lo, m_hi) x [n_lo, n_hi), moved to the origin
  const float* __restrict__ A = @A@ + (size_t)__eas_m_lo * K;
  const float* __restrict__ B = @B@ + __eas_n_lo;
  float* __restrict__ C = @C@ + (size_t)__eas_m_lo * ldb + __eas_n_lo;
  const int M = (int)(__eas_m_hi - __eas_m_lo), N = (int)(__eas_n_hi - __eas_n_lo);
  __shared__ __attribute__((aligned(1024))) float smem[NSTAGE * STF];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-contiguous, M-grouped tile order
  const int tilesM = (M + BM - 1) / BM, tilesN = (N + BN - 1) / BN, T = tilesM * tilesN;
  const int w = blockIdx.x;
  const int t = (T % 8 == 0) ? (w % 8) * (T / 8) + w / 8 : w;
  constexpr int GROUP_M = 4;
  const int gsize = GROUP_M * tilesN, g = t / gsize, first_m = g * GROUP_M;
  const int gm = min(tilesM - first_m, GROUP_M);
  const int m0 = (first_m + (t % gsize) % gm) * BM, n0 = ((t % gsize) / gm) * BN;
  const bool dma_ok = (K % 4 == 0) && (ldb % 4 == 0) && ((((uint64_t)A) | ((uint64_t)B)) % 16 == 0) &&
                      ((uint64_t)M * K * 4 < (1ull << 31)) && (((uint64_t)(K - 1) * ldb + N) * 4 < (1ull << 31));
  if (!dma_ok) {
    // guard for operands the launch plan could not see: one f32 dot product per element
    for (int e = tid; e < BM * BN; e += 512) {
      const int row = m0 + e / BN, col = n0 + e % BN;
      if (row >= M || col >= N) continue;
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc = __builtin_fmaf(A[(size_t)row * K + k], B[(size_t)k * ldb + col], acc);
      C[(size_t)row * ldb + col] = acc;
    }
    return;
  }
  if (wave >= 4) {
    // producer: the DMA (1 KB per instruction, 4 A + 4 B per wave per stage, q = 4 pw + i)
    //   A stage [128 rows][32 k]: rows 8q + lane/8, chunk lane%8 stored at chunk ^ ((row/2)%8)
    //   B stage [32 k][128 n]:    rows 2q + lane/32, chunk lane%32 stored at chunk ^ 8((row/16)%2)
    // Rows past M and columns past N load zeros (they are never stored), so every address a load
    // reads, lane offset plus stage offset, lies inside A or B.  The last stage of a K that is not
    // a multiple of BK loads zeros past K; stages past K load zeros into a slot nobody reads, so
    // every stage issues 8 loads and the count at each barrier is the same.
    const int pw = wave - 4;
    const eas_rsrc ra = eas_make_rsrc(A, (uint32_t)M * (uint32_t)K * 4u);
    const eas_rsrc rb = eas_make_rsrc(B, ((uint32_t)(K - 1) * (uint32_t)ldb + (uint32_t)N) * 4u);
    const uint32_t lds0 = (uint32_t)(size_t)(EAS_LDS float*)smem;
    constexpr int KLAST = K - (KT - 1) * BK;  // k extent of the last stage
    uint32_t a_off[4], b_off[4], a_tail[4], b_tail[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = pw * 4 + i;
      const int r = 8 * q + (lane >> 3), lc = (lane & 7) ^ ((r >> 1) & 7);
      a_off[i] = m0 + r < M ? ((uint32_t)(m0 + r) * (uint32_t)K + (uint32_t)(lc * 4)) * 4u : 0x80000000u;
      a_tail[i] = lc * 4 >= KLAST ? 0x80000000u : a_off[i];
      const int rr = 2 * q + (lane >> 5), lcb = (lane & 31) ^ (8 * ((rr >> 4) & 1));
      b_off[i] = n0 + lcb * 4 < N ? (uint32_t)(n0 + lcb * 4) * 4u + (uint32_t)rr * (uint32_t)ldb * 4u : 0x80000000u;
      b_tail[i] = rr >= KLAST ? 0x80000000u : b_off[i];
    }
    auto dma = [&](int kt) {
      const uint32_t st = lds0 + (uint32_t)((kt % NSTAGE) * STF) * 4u;
      const uint32_t sa = (uint32_t)(kt * BK) * 4u, sb = (uint32_t)(kt * BK) * (uint32_t)ldb * 4u;
      if (kt >= KT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          eas_dma16s(ra, 0x80000000u, 0u, st + (pw * 4 + i) * 1024);
          eas_dma16s(rb, 0x80000000u, 0u, st + AST * 4 + (pw * 4 + i) * 1024);
        }
      } else if (K % BK != 0 && kt == KT - 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          eas_dma16s(ra, a_tail[i], sa, st + (pw * 4 + i) * 1024);
          eas_dma16s(rb, b_tail[i], sb, st + AST * 4 + (pw * 4 + i) * 1024);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          eas_dma16s(ra, a_off[i], sa, st + (pw * 4 + i) * 1024);
          eas_dma16s(rb, b_off[i], sb, st + AST * 4 + (pw * 4 + i) * 1024);
        }
      }
    };
    // one barrier per stage, as many as the consumers
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) dma(p);
    __builtin_amdgcn_s_waitcnt(EAS_WAITVM(16));  // stage 0 landed (stages 1 and 2 may be in flight)
    __syncthreads();
    for (int kt = 0; kt + 1 < KT; ++kt) {
      __builtin_amdgcn_s_waitcnt(EAS_WAITVM(8));  // stage kt+1 landed (stage kt+2 may be in flight)
      __syncthreads();
      dma(kt + NSTAGE - 1);  // the slot of stage kt-1, whose fragments every consumer has read
    }
    __builtin_amdgcn_s_waitcnt(EAS_WAITVM(0));
    return;
  }
  const int wm = wave >> 1, wn = wave & 1;
  // MFMA step s (0..15) of a stage takes k = s + 16 c for lane half c = lane/32
  const int c = lane >> 5;
  int fa[2][4], fb[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ai = wm * 64 + i * 32 + (lane & 31);
#pragma unroll
    for (int u = 0; u < 4; ++u) fa[i][u] = ai * BK + (((4 * c + u) ^ ((ai >> 1) & 7)) * 4);
    const int bj = wn * 64 + i * 32 + (lane & 31);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int row = s + 16 * c;
      fb[i][s] = AST + row * BN + (((bj >> 2) ^ (8 * ((row >> 4) & 1))) * 4) + (bj & 3);
    }
  }
  eas_f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (eas_f32x16){};
  // Fragments are read one stage ahead, interleaved with the MFMAs: at the barrier of stage kt
  // the producers' DMA of stage kt+1 has landed; after it the wave issues stage kt's 64 MFMAs
  // from the register set read one stage earlier and, between them (sched_group_barrier), every
  // fragment read of stage kt+1 into the other set.  After this barrier the producers refill the
  // slot of stage kt-1, whose fragments every consumer read (and waited for, at the barrier of
  // stage kt-1) before it.
  auto read_stage = [&](int kt, eas_f32x4 (&a)[2][4], float (&b)[2][16]) {
    const float* st = smem + (kt % NSTAGE) * STF;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int u = 0; u < 4; ++u) a[i][u] = *(const eas_f32x4*)(st + fa[i][u]);
#pragma unroll
      for (int s = 0; s < 16; ++s) b[i][s] = st[fb[i][s]];
    }
  };
  auto mfmas = [&](const eas_f32x4 (&a)[2][4], const float (&b)[2][16]) {
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s >> 2][s & 3], b[j][s], acc[i][j], 0, 0, 0);
  };
  // a stage that is followed by another (KT - 1 of them, each with the barrier the producers match)
  auto step = [&](int kt, const eas_f32x4 (&a)[2][4], const float (&b)[2][16], eas_f32x4 (&na)[2][4],
                  float (&nb)[2][16]) {
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_stage(kt + 1, na, nb);
    mfmas(a, b);
    // one LDS read after each of the first 40 MFMAs
#pragma unroll
    for (int s = 0; s < 40; ++s) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 24, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  __syncthreads();  // stage 0 landed
  eas_f32x4 a0[2][4], a1[2][4];
  float b0[2][16], b1[2][16];
  read_stage(0, a0, b0);
  int kt = 0;
  for (; kt + 2 < KT; kt += 2) {  // two stages per iteration: the register sets alternate
    step(kt, a0, b0, a1, b1);
    step(kt + 1, a1, b1, a0, b0);
  }
  if constexpr (KT % 2 == 0) {
    step(KT - 2, a0, b0, a1, b1);
    mfmas(a1, b1);
  } else {
    mfmas(a0, b0);
  }
  // lane l, register r holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + (r / 4) * 8 + (lane >> 5) * 4 + (r % 4);
        const int col = n0 + wn * 64 + j * 32 + (lane & 31);
        if (row < M && col < N) C[(size_t)row * ldb + col] = acc[i][j][r];
      }
}
"""

TILE = (256, 256)  # BM, BN
TILE_F32 = (64, 64)
THREADS = 256
PP_THREADS = 512  # the 8-wave (ping-pong) entry of f16 GEMMs
T128_THREADS = 512  # the smaller-tile entries of f16 GEMMs: 4 consumer + 4 producer waves
F32_THREADS = 512  # both fp32 entries: 4 consumer + 4 producer waves
SKINNY_M = 128  # launches of at most this many rows run the skinny path: one workgroup per SKINNY_N columns
SKINNY_N = 64
# MFMA shape of the 8-wave and smaller-tile entries' bodies: 16 (v_mfma_f32_16x16x32, the default) or
# 32 (v_mfma_f32_32x32x16).  Measured on MI355X with random inputs, where the part runs
# power-limited: 16 x 16 x 32 is 2.5-5 % faster on the 8-wave entry (4096³ f16 1172-1181 ->
# 1219-1222 TFLOP/s, 8192³ 1271-1277 -> 1331-1335), since it moves fewer accumulator bytes per
# flop, and 2.5-4.7 % on the 128 x 128 entry (2048³ 24.32 -> 23.17 µs, 256 x 14336 x 4096
# 40.96 -> 39.95 µs by rocprof).
def pp_mfma() -> int:
    """``EAS_HIP_GEMM_MFMA``: 16 (default) or 32, read each time a GEMM source is emitted."""
    v = os.environ.get("EAS_HIP_GEMM_MFMA", "16").strip() or "16"
    if v not in ("16", "32"):
        raise ValueError(f"EAS_HIP_GEMM_MFMA must be 16 or 32, got {v!r}")
    return int(v)


def emit_gemm(ir: IRModule, block: int, spec: GemmSpec) -> Lowered:
    bm, bn = TILE
    # Parameters keep the user's order (kernel arguments are positional) but get
    # private names, so user names cannot collide with the template's locals.
    params = []
    pname = {}
    for i, arg in enumerate(ir.args):
        pname[arg.name] = f"__eas_a{i}"
        if arg.kind == "buffer":
            const = "" if arg.name == spec.c else "const "
            params.append(f"{const}{ctype(arg.dtype)}* __restrict__ __eas_a{i}")
        else:
            params.append(f"const {ctype(arg.dtype)} __eas_a{i}")
    params += ["const uint32_t __eas_m_lo", "const uint32_t __eas_m_hi", "const uint32_t __eas_n_lo",
               "const uint32_t __eas_n_hi"]
    # the DMA bodies copy A and B as they lie in HBM: both must already be the MFMA operand type
    op_in = spec.a_dtype == spec.op_dtype and spec.b_dtype == spec.op_dtype
    assert SKINNY_N == 64, "the skinny path's tile width is fixed by its LDS layout"
    if spec.f32:
        bm, bn = TILE_F32
    subs = {
        "@NAME@": ir.name,
        "@SKINNY_M@": str(SKINNY_M),
        "@PARAMS@": ",\n    ".join(params),
        "@K@": str(spec.K),
        "@OP_IN@": "true" if op_in else "false",
        "@AT@": ctype(spec.a_dtype),
        "@BT@": ctype(spec.b_dtype),
        "@CT@": ctype(spec.c_dtype),
        "@A@": pname[spec.a],
        "@B@": pname[spec.b],
        "@C@": pname[spec.c],
        "@LDB@": pname[spec.n_sym],
        "@PP_MI@": str(pp_mfma()),
    }
    src = _DMA_HELPERS + (_TEMPLATE_F32 + _TEMPLATE_F32_T128 if spec.f32 else _OP_TYPES[spec.op_dtype] + _TEMPLATE)
    pingpong = op_in and not spec.f32 and spec.K % 2 == 0  # odd K: rows of A are not 4-byte aligned
    if pingpong:
        src += _TEMPLATE_PP_ENTRY
    for k, v in subs.items():
        src = src.replace(k, v)
    header = (f"// Lifted from eas kernel `{ir.name}`: proven dense GEMM C[M,N] = A[M,{spec.K}] @ B[{spec.K},N]\n"
              f"// (A={spec.a}, B={spec.b}, C={spec.c}, M={spec.m_sym}, N={spec.n_sym}, reference tile "
              f"{spec.TM}x{spec.TN} rows on program_id({spec.row_axis})).\n")
    threads = F32_THREADS if spec.f32 else THREADS
    geo = Geometry("gemm", ir.name, block, threads, params={
        "m_sym": spec.m_sym, "n_sym": spec.n_sym, "K": spec.K, "TM": spec.TM, "TN": spec.TN,
        "row_axis": spec.row_axis, "BM": bm, "BN": bn, "threads": threads,
        "skinny_m": 0 if spec.f32 else SKINNY_M, "skinny_n": SKINNY_N, "row_base": spec.row_base,
        "col_base": spec.col_base,
        "col_masked": spec.col_masked,
        "pp_entry": f"{ir.name}__pp" if pingpong else None, "pp_threads": PP_THREADS,
        "t128_entry": f"{ir.name}__t128" if (pingpong or spec.f32) else None, "f32": spec.f32,
        "t128_threads": F32_THREADS if spec.f32 else T128_THREADS,
        "t128x256_entry": f"{ir.name}__t128x256" if pingpong else None,
        "t128x64_entry": f"{ir.name}__t128x64" if pingpong else None,
        "t64_entry": f"{ir.name}__t64x64" if pingpong else None,
        "a": spec.a, "b": spec.b, "c": spec.c, "out_dtype": spec.c_dtype.value,
        "op_dtype": "f32" if spec.f32 else spec.op_dtype.value})
    return Lowered(PRELUDE + header + src, block, "thread", geo)
