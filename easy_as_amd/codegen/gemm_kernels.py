"""gfx950 MFMA GEMM emitted for kernels that ``gemm_lift`` proved to be dense GEMMs.

Design (MI355X / CDNA4):

* workgroup tile BM x BN with BK = 64, waves arranged WM x WN; each wave owns a
  (BM/WM) x (BN/WN) block of 32x32 accumulators fed by
  ``v_mfma_f32_32x32x16_f16`` (A: 8 consecutive k per lane, B: 8 consecutive
  k per lane, f32 accumulate in AGPRs);
* A and B stream global -> registers -> LDS, double buffered (one barrier per
  k-tile, next tile's loads issued before the current tile's MFMAs);
* B is row-major (k, n) in HBM but MFMA wants k contiguous per lane: each
  thread loads an 8(k) x 8(n) block (eight 16-byte row loads) and transposes it
  in registers, so LDS holds B as [n][k]; the lane -> block map puts the k-group
  fastest so every 16-lane LDS write group covers 256 distinct bytes;
* LDS rows are padded by 16 bytes (pitch BK+8 halves) so the 32 rows a
  fragment read touches fall in distinct banks;
* tile order is XCD aware: workgroup w runs on XCD w % 8, so each XCD gets a
  contiguous range of tiles, grouped 4 tile-rows high for L2 reuse;
* interior tiles take a branch-free path; edge tiles and the K tail use masked
  loads (zero fill) and masked stores.

The kernel computes C[m, n] for m < m_eff, n < n_eff (hidden arguments: the
rectangle the reference launch covers).  Rows of A have length K (a compile-
time constant); B and C rows have the scalar argument ``ldb`` as stride.
"""

from __future__ import annotations

from ..ir import DType, IRModule
from .gemm_lift import GemmSpec
from .hip import PRELUDE, Geometry, Lowered, ctype

_TEMPLATE = r"""
typedef _Float16 eas_h8 __attribute__((ext_vector_type(8)));
typedef float eas_f32x16 __attribute__((ext_vector_type(16)));

template <typename T> static __device__ __forceinline__ eas_h8 eas_load8(const T* p);
template <> __device__ __forceinline__ eas_h8 eas_load8<_Float16>(const _Float16* p) { return *(const eas_h8*)p; }
template <> __device__ __forceinline__ eas_h8 eas_load8<float>(const float* p) {
  const eas_f32x4 lo = *(const eas_f32x4*)p, hi = *(const eas_f32x4*)(p + 4);
  eas_h8 v;
  v[0] = (_Float16)lo[0]; v[1] = (_Float16)lo[1]; v[2] = (_Float16)lo[2]; v[3] = (_Float16)lo[3];
  v[4] = (_Float16)hi[0]; v[5] = (_Float16)hi[1]; v[6] = (_Float16)hi[2]; v[7] = (_Float16)hi[3];
  return v;
}

extern "C" __global__ __launch_bounds__(@THREADS@) void @NAME@(
    @PARAMS@) {
  constexpr int BM = @BM@, BN = @BN@, BK = 64, WM = @WM@, WN = @WN@, K = @K@;
  constexpr int PITCH = BK + 8, NTHREADS = WM * WN * 64, TI = BM / WM / 32, TJ = BN / WN / 32;
  constexpr int KC = BK / 8, A_IT = BM * BK / 8 / NTHREADS, NBLK = BK * BN / 64;
  constexpr int B_IT = (NBLK + NTHREADS - 1) / NTHREADS;
  typedef @AT@ AT;
  typedef @BT@ BT;
  const AT* __restrict__ A = @A@;
  const BT* __restrict__ B = @B@;
  @CT@* __restrict__ C = @C@;
  const int ldb = (int)@LDB@;
  const int M = (int)__eas_m_eff, N = (int)__eas_n_eff;
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * PITCH];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  // XCD-contiguous, M-grouped tile order
  const int tilesM = (M + BM - 1) / BM, tilesN = (N + BN - 1) / BN, T = tilesM * tilesN;
  const int w = blockIdx.x;
  const int t = (T % 8 == 0) ? (w % 8) * (T / 8) + w / 8 : w;
  constexpr int GROUP_M = 4;
  const int gsize = GROUP_M * tilesN, g = t / gsize, first_m = g * GROUP_M;
  const int gm = min(tilesM - first_m, GROUP_M);
  const int ty = first_m + (t % gsize) % gm, tx = (t % gsize) / gm;
  const int m0 = ty * BM, n0 = tx * BN;
  // 16-byte vector loads need aligned rows and base pointers; anything else takes the masked path
  const bool mn_full = (m0 + BM <= M) && (n0 + BN <= N) && (ldb % 8 == 0) && (K % 8 == 0) &&
                       ((((uint64_t)A) | ((uint64_t)B)) % 32 == 0);

  eas_h8 ra[A_IT], rb[B_IT][8];
  auto gload_fast = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + NTHREADS * i, row = c / KC, kc = c % KC;
      ra[i] = eas_load8<AT>(A + (size_t)(m0 + row) * K + k0 + kc * 8);
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int blk = tid + NTHREADS * i, kg = blk % KC, nc = blk / KC;
      if (NBLK % NTHREADS != 0 && blk >= NBLK) break;
#pragma unroll
      for (int r = 0; r < 8; ++r) rb[i][r] = eas_load8<BT>(B + (size_t)(k0 + kg * 8 + r) * ldb + n0 + nc * 8);
    }
  };
  auto gload_masked = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + NTHREADS * i, row = c / KC, kc = c % KC;
      const int gm_ = m0 + row, gk = k0 + kc * 8;
      eas_h8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (gm_ < M && gk + e < K) ? (_Float16)A[(size_t)gm_ * K + gk + e] : (_Float16)0.0f;
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int blk = tid + NTHREADS * i, kg = blk % KC, nc = blk / KC;
      if (NBLK % NTHREADS != 0 && blk >= NBLK) break;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int gk = k0 + kg * 8 + r, gn = n0 + nc * 8;
        eas_h8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (gk < K && gn + e < N) ? (_Float16)B[(size_t)gk * ldb + gn + e] : (_Float16)0.0f;
        rb[i][r] = v;
      }
    }
  };
  auto gload = [&](int k0) {
    if (mn_full && k0 + BK <= K) gload_fast(k0);
    else gload_masked(k0);
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int c = tid + NTHREADS * i, row = c / KC, kc = c % KC;
      *(eas_h8*)(&As[buf][row * PITCH + kc * 8]) = ra[i];
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
        *(eas_h8*)(&Bs[buf][(nc * 8 + j) * PITCH + kg * 8]) = col;
      }
    }
  };

  eas_f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = (eas_f32x16){};

  constexpr int KT = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      eas_h8 a[TI], b[TJ];
      const int kk = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TI; ++i) a[i] = *(const eas_h8*)&As[buf][(wm * (BM / WM) + i * 32 + (lane & 31)) * PITCH + kk];
#pragma unroll
      for (int j = 0; j < TJ; ++j) b[j] = *(const eas_h8*)&Bs[buf][(wn * (BN / WN) + j * 32 + (lane & 31)) * PITCH + kk];
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(buf ^ 1);
    __syncthreads();
  }
  // epilogue: lane l, register r of a 32x32 tile holds (row 8*(r/4) + 4*(l/32) + r%4, col l%32)
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * (BM / WM) + i * 32 + (r / 4) * 8 + (lane >> 5) * 4 + (r % 4);
        const int col = n0 + wn * (BN / WN) + j * 32 + (lane & 31);
        if (mn_full || (row < M && col < N)) C[(size_t)row * ldb + col] = (@CT@)acc[i][j][r];
      }
}
"""

# Tile configurations (BM, BN, WM, WN); measured on MI355X, see the DESIGN notes.
CONFIGS = {
    "large": (256, 256, 2, 2),
    "medium": (128, 256, 2, 2),
}


def emit_gemm(ir: IRModule, block: int, spec: GemmSpec) -> Lowered:
    bm, bn, wm, wn = CONFIGS["large"]
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
    params += ["const uint32_t __eas_m_eff", "const uint32_t __eas_n_eff"]
    subs = {
        "@NAME@": ir.name,
        "@THREADS@": str(wm * wn * 64),
        "@PARAMS@": ",\n    ".join(params),
        "@BM@": str(bm),
        "@BN@": str(bn),
        "@WM@": str(wm),
        "@WN@": str(wn),
        "@K@": str(spec.K),
        "@AT@": ctype(spec.a_dtype),
        "@BT@": ctype(spec.b_dtype),
        "@CT@": ctype(spec.c_dtype),
        "@A@": pname[spec.a],
        "@B@": pname[spec.b],
        "@C@": pname[spec.c],
        "@LDB@": pname[spec.n_sym],
    }
    src = _TEMPLATE
    for k, v in subs.items():
        src = src.replace(k, v)
    header = (f"// Lifted from eas kernel `{ir.name}`: proven dense GEMM C[M,N] = A[M,{spec.K}] @ B[{spec.K},N]\n"
              f"// (A={spec.a}, B={spec.b}, C={spec.c}, M={spec.m_sym}, N={spec.n_sym}, reference tile "
              f"{spec.TM}x{spec.TN} rows on program_id({spec.row_axis})).\n")
    geo = Geometry("gemm", ir.name, block, wm * wn * 64, params={
        "m_sym": spec.m_sym, "n_sym": spec.n_sym, "K": spec.K, "TM": spec.TM, "TN": spec.TN,
        "row_axis": spec.row_axis, "BM": bm, "BN": bn, "threads": wm * wn * 64,
        "a": spec.a, "b": spec.b, "c": spec.c, "out_dtype": spec.c_dtype.value})
    return Lowered(PRELUDE + header + src, block, "thread", geo)
