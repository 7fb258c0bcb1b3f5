// Skinny quantized matmul, M <= 16 rows: out[M,N] = x[M,K] . deq(W[N,K])^T.
//
// One kernel family covers the reference's M=1 decode path (mx.quantized_matmul
// -> MLX qmv_fast, mlxturbo/kernels/dispatch.py:317-327) and its M=2..16
// verify window (kernels/qmv_small_m.py:289-335, fast_qmm.py:334-374,
// kernels/qmv_wide_nocap.py:240-288).
//
// The packed weights stream from HBM once; everything is laid out for that
// stream, for the VMEM instruction count and for the VALU cost of exact
// dequantization, which measurement showed to be the three limiters:
//
//  * A workgroup owns a tile of 16 weight rows; its NW waves split the tile's
//    K range into contiguous slices of whole steps.  Lane (r = lane & 15,
//    c = lane >> 4) reads row r.  A step covers 4*GPL quantization groups of
//    each row; lane c owns groups c, c+4, ... of the step, so one scale/bias
//    pair serves GS codes of the lane (4 VALU ops per group).
//  * Weights, scales and biases are read with buffer loads whose descriptor
//    is rebuilt per step in scalar registers.  A step beyond the wave's slice
//    gets num_records = 0, so its loads return zeros without touching memory;
//    that keeps the PF-stage prefetch pipeline free of conditional loads
//    (vmcnt waits stay exact).  Rows past N are past num_records as well.
//  * x (M rows) lives in LDS when it fits: each wave copies its own K slice
//    (no workgroup barrier before the main loop) and reads MFMA A fragments
//    with ds_read_b128.  Lanes whose A row is >= M read row M-1: it only
//    fills output rows that are never stored, since the rows of an MFMA
//    product are independent.  When x does not fit, fragments come from
//    global memory in the same order.
//  * Dequantization is the exact fma_mix trick of mq_common.h, rounded to T
//    per weight (bit-exact MLX dequantization); the packed T pairs are the
//    B operand of v_mfma_f32_16x16x32 (32 k x 16 rows).  A and B use the same
//    lane -> k mapping, so the permuted k order inside each MFMA is harmless.
//    Scales with |s| >= 2^100 (never seen in real checkpoints) switch the
//    whole step, wave-uniformly, to a plain float route.
//  * The NW partial 16x16 tiles are summed in LDS in wave order and rounded
//    once.  The K decomposition depends on (N, K, bits, group_size) only, so
//    each output row is bit-identical for every M (the property the
//    reference tests for its small-M kernel: bench/test_qmm_smallm.py:70-85).
#pragma once
#include "mq_common.h"

namespace mq {

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) unsigned char lds_u8;

// Buffer resource for a raw (unstructured) byte range.  Word 3 is the gfx9
// default for 32-bit data; out-of-range loads return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// v_perm selector moving 16-bit half h (0..3 of the 64-bit pair {hi:lo}) to
// where a float conversion wants it: bf16 -> bits 16..31 (the float's bits),
// f16 -> bits 0..15.  Selector byte 0x0c yields 0x00.
template <int DT>
__device__ __forceinline__ uint32_t half_selector(int h) {
  const uint32_t b0 = 2u * (uint32_t)h, b1 = b0 + 1u;
  if constexpr (DT == kBF16) return 0x0c0cu | (b0 << 16) | (b1 << 24);
  else return b0 | (b1 << 8) | 0x0c0c0000u;
}

template <int DT>
__device__ __forceinline__ float selected_to_f32(uint32_t v) {
  if constexpr (DT == kBF16) return __uint_as_float(v);
  else return (float)bitcast<_Float16>((uint16_t)v);
}

template <int BITS, int GS, int GPL>
struct QmvGeom {
  static constexpr int GB = GS * BITS / 8;         // bytes of one group of one row
  static constexpr int LPG = GB / 16;              // 16-byte loads per group
  static constexpr int STEPG = 4 * GPL;            // groups per row per step
  static constexpr int STEPB = STEPG * GB;         // weight bytes per row per step
  static constexpr int STEPK = STEPG * GS;         // codes per step
  static constexpr int NSV = STEPG / 2;            // scale dwords per row per step
  static constexpr int CPL = 128 / BITS;           // codes per 16-byte load
  static constexpr int MPL = (BITS == 4) ? 4 : 2;  // MFMAs per 16-byte load (8 codes each)
  static_assert(LPG >= 1, "a group must span at least one 16-byte load");
  static_assert(NSV == 2 || NSV % 4 == 0, "scale vector must be 8 bytes or whole 16-byte loads");
};

// Bytes per LDS row of the x copy: the K range padded to whole steps, plus 16
// bytes so consecutive rows start in different banks.
__host__ __device__ inline int qmv_x_stride(int K, int stepk) {
  return 2 * (((K + stepk - 1) / stepk) * stepk) + 16;
}

// Launch geometry of the skinny kernel for one (bits, group_size): groups per
// lane per step, waves per workgroup, pipeline stages.  Fixed per format (not
// per M), so every output row is computed in the same order for every M.
template <int BITS, int GS>
struct QmvConf {
  static constexpr int GPL = (BITS == 4 && GS == 32) ? 4 : (BITS == 8 && GS >= 64) ? 1 : 2;
  static constexpr int NW = 4;
  static constexpr int PF = 2;
};

// Largest x copy (M rows) kept in LDS; beyond it fragments are read from global memory.
constexpr size_t kQmvMaxXLds = 64 * 1024;

// Row sources of a tile: where the A rows (x) come from and where outputs go.
// Dense: A row m is x row m; output (m, column n0 + nn).
struct DenseRows {
  const uint16_t* x;
  uint16_t* out;
  int64_t ldx, ldo;
  int n0;
  __device__ __forceinline__ const uint16_t* xrow(int m) const { return x + (int64_t)m * ldx; }
  __device__ __forceinline__ void store(int m, int nn, uint16_t v) const {
    out[(int64_t)m * ldo + n0 + nn] = v;
  }
};

// One 16-row weight tile (rows n0 .. n0+rows-1 of a [*, K] quantized matrix
// whose row n0 starts at wt / st / bt) times M <= 16 A rows.  Called by every
// thread of a 64*NW-thread workgroup; dynamic LDS holds the x copy.
template <int DT, int BITS, int GS, int GPL, int NW, int PF, bool XLDS, class Rows>
__device__ __forceinline__ void qmv_tile(const char* __restrict__ wt, const char* __restrict__ st,
                                         const char* __restrict__ bt, int rows, int M, int K,
                                         const Rows& src, unsigned char* qmv_smem,
                                         f32x4 (*red)[64], bool copy_x = true) {
  using Gm = QmvGeom<BITS, GS, GPL>;
  constexpr int GB = Gm::GB, LPG = Gm::LPG, STEPG = Gm::STEPG, STEPB = Gm::STEPB;
  constexpr int STEPK = Gm::STEPK, NSV = Gm::NSV, CPL = Gm::CPL, MPL = Gm::MPL;
  using T = T16<DT>;
  struct Stage {
    u32x4 w[GPL][LPG];
    uint32_t s[NSV], b[NSV];
  };
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, c = lane >> 4;
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const int G = K / GS;
  const uint32_t sRowB = (uint32_t)G * 2;
  const uint32_t w_nrec = (uint32_t)(rows - 1) * rowB + STEPB;
  const uint32_t s_nrec = (uint32_t)(rows - 1) * sRowB + STEPG * 2;
  const uint32_t wofs = (uint32_t)r * rowB + (uint32_t)c * GB;
  const uint32_t sofs = (uint32_t)r * sRowB;
  const uint32_t sel = half_selector<DT>(c);

  const int nsteps = (G + STEPG - 1) / STEPG;
  const int full = G / STEPG;                 // steps with every group inside K
  const int sb = (int)((int64_t)nsteps * wave / NW);
  const int se = (int)((int64_t)nsteps * (wave + 1) / NW);
  const int fe = se < full ? se : full;      // pipelined (unchecked) steps: [sb, fe)

  auto load = [&](Stage& s, int t, bool live) {
    const auto rw = make_rsrc(wt + (int64_t)t * STEPB, live ? w_nrec : 0u);
    const auto rs = make_rsrc(st + (int64_t)t * STEPG * 2, live ? s_nrec : 0u);
    const auto rb = make_rsrc(bt + (int64_t)t * STEPG * 2, live ? s_nrec : 0u);
#pragma unroll
    for (int j = 0; j < GPL; ++j)
#pragma unroll
      for (int h = 0; h < LPG; ++h)
        s.w[j][h] = __builtin_amdgcn_raw_buffer_load_b128(rw, wofs + j * 4 * GB + h * 16, 0, 0);
    if constexpr (NSV == 2) {
      const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rs, sofs, 0, 0);
      const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(rb, sofs, 0, 0);
      s.s[0] = a[0]; s.s[1] = a[1]; s.b[0] = q[0]; s.b[1] = q[1];
    } else {
#pragma unroll
      for (int v = 0; v < NSV / 4; ++v) {
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, sofs + 16 * v, 0, 0);
        const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rb, sofs + 16 * v, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) { s.s[4 * v + e] = a[e]; s.b[4 * v + e] = q[e]; }
      }
    }
  };

  // ---- x: this wave's K slice into LDS (zero-padded past K) -----------------
  const int xs = qmv_x_stride(K, STEPK);
  const int kb = sb * STEPK, ke = se * STEPK;
  const int xr = min(r, M - 1);
  const lds_u8* xl = (const lds_u8*)qmv_smem + xr * xs;       // XLDS: A row of this lane
  const uint16_t* xg = src.xrow(xr);                           // !XLDS: same, in global memory
  constexpr int XB = 4;                                        // x pieces per lane per batch
  const int pw = (ke - kb) / 8;                                // 16-byte pieces per row
  const int npieces = (XLDS && copy_x) ? M * pw : 0;
  u32x4 xp[XB];
  auto x_fetch = [&](int base) {
#pragma unroll
    for (int q = 0; q < XB; ++q) {
      const int i = base + q * 64;
      xp[q] = (u32x4){0u, 0u, 0u, 0u};
      if (i < npieces) {
        const int m = i / pw, k = kb + 8 * (i - m * pw);
        if (k < K) xp[q] = *reinterpret_cast<const u32x4*>(src.xrow(m) + k);
      }
    }
  };
  auto x_store = [&](int base) {
#pragma unroll
    for (int q = 0; q < XB; ++q) {
      const int i = base + q * 64;
      if (i < npieces) {
        const int m = i / pw, k = kb + 8 * (i - m * pw);
        *(lds_u32x4*)((lds_u8*)qmv_smem + m * xs + 2 * k) = xp[q];
      }
    }
  };
  if constexpr (XLDS) x_fetch(lane);

  Stage S[PF];
#pragma unroll
  for (int i = 0; i < PF - 1; ++i) load(S[i], sb + i, sb + i < fe);

  if (XLDS && copy_x) {
    x_store(lane);
    for (int base = lane + XB * 64; base < npieces; base += XB * 64) {
      x_fetch(base);
      x_store(base);
    }
    // each wave reads only the slice it wrote itself
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};

  // A fragment of the MFMA covering codes [k, k+8) of this lane.  Global x
  // fragments past K are zeroed (LDS rows are zero-padded there).
  auto afrag = [&](int k, bool checked) -> u32x4 {
    if constexpr (XLDS) {
      (void)checked;
      return *(const lds_u32x4*)(xl + 2 * k);
    } else {
      if (checked && k >= K) return (u32x4){0u, 0u, 0u, 0u};
      return *reinterpret_cast<const u32x4*>(xg + k);
    }
  };

  auto compute = [&](const Stage& s, int t, bool checked) {
    float sf[GPL], bf[GPL];
    bool big = false;
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      sf[j] = selected_to_f32<DT>(__builtin_amdgcn_perm(s.s[2 * j + 1], s.s[2 * j], sel));
      bf[j] = selected_to_f32<DT>(__builtin_amdgcn_perm(s.b[2 * j + 1], s.b[2 * j], sel));
      if (checked && t * STEPG + c + 4 * j >= G) { sf[j] = 0.f; bf[j] = 0.f; }
      big |= needs_plain(sf[j]);
    }
    const int kt = t * STEPK + c * GS;
    if (__builtin_amdgcn_ballot_w64(big) == 0) {
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const GroupScale g = make_group(sf[j], bf[j]);
#pragma unroll
        for (int h = 0; h < LPG; ++h)
#pragma unroll
          for (int p = 0; p < MPL; ++p) {
            uint32_t bo[4];
            if constexpr (BITS == 4) {
              deq4_word<DT>(s.w[j][h][p], g, bo);
            } else {
              deq8_word<DT>(s.w[j][h][2 * p], g, bo);
              deq8_word<DT>(s.w[j][h][2 * p + 1], g, bo + 2);
            }
            const u32x4 a = afrag(kt + j * 4 * GS + h * CPL + 8 * p, checked);
            acc = T::mfma(a, (u32x4){bo[0], bo[1], bo[2], bo[3]}, acc);
          }
      }
    } else {
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const GroupScale g = make_group(sf[j], bf[j]);
#pragma unroll
        for (int h = 0; h < LPG; ++h)
#pragma unroll
          for (int p = 0; p < MPL; ++p) {
            uint32_t bo[4];
            if constexpr (BITS == 4) {
              deq_word_plain<DT, 4>(s.w[j][h][p], g, bo);
            } else {
              deq_word_plain<DT, 8>(s.w[j][h][2 * p], g, bo);
              deq_word_plain<DT, 8>(s.w[j][h][2 * p + 1], g, bo + 2);
            }
            const u32x4 a = afrag(kt + j * 4 * GS + h * CPL + 8 * p, checked);
            acc = T::mfma(a, (u32x4){bo[0], bo[1], bo[2], bo[3]}, acc);
          }
      }
    }
  };

  // ---- main loop: PF-stage pipeline over the unchecked steps --------------
  for (int t = sb; t < fe; t += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int tl = t + i + PF - 1;
      load(S[(i + PF - 1) % PF], tl, tl < fe);
      if (t + i < fe) compute(S[i], t + i, false);
    }
  }
  // ---- ragged tail: at most one step; groups past K are zeroed ------------
  if (fe < se) {
    Stage s;
    load(s, fe, true);
#pragma unroll
    for (int j = 0; j < GPL; ++j)
      if (fe * STEPG + c + 4 * j >= G)
#pragma unroll
        for (int h = 0; h < LPG; ++h) s.w[j][h] = (u32x4){0u, 0u, 0u, 0u};
    compute(s, fe, true);
  }

  // ---- sum the waves' partial tiles in wave order, round once -------------
  // lane l holds D[4*(l>>4)+v][l&15]: output row 4c+v, column n0 + r
  if constexpr (NW == 1) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * c + v;
      if (m < M && r < rows) src.store(m, r, T::round1(acc[v]));
    }
  } else {
    red[wave][lane] = acc;
    __syncthreads();
    for (int tt = threadIdx.x; tt < 256; tt += 64 * NW) {
      const int mm = tt >> 4, nn = tt & 15;
      const int sl = ((mm >> 2) << 4) | nn, v = mm & 3;
      float sum = red[0][sl][v];
#pragma unroll
      for (int q = 1; q < NW; ++q) sum += red[q][sl][v];
      if (mm < M && nn < rows) src.store(mm, nn, T::round1(sum));
    }
    __syncthreads();
  }
}

// grid.x = ceil(N / 16) tiles, block = 64 * NW threads.
// Dynamic LDS: XLDS ? M * qmv_x_stride(K, STEPK) : 0 bytes.
template <int DT, int BITS, int GS, int GPL, int NW, int PF, bool XLDS>
__global__ __launch_bounds__(64 * NW) void qmv_kernel(const uint16_t* __restrict__ x,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      uint16_t* __restrict__ out, int M, int N,
                                                      int K, int64_t ldx, int64_t ldo) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  __shared__ f32x4 red[NW][64];
  const int n0 = blockIdx.x * 16;
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K / GS) * 2;
  const DenseRows src{x, out, ldx, ldo, n0};
  qmv_tile<DT, BITS, GS, GPL, NW, PF, XLDS>(
      reinterpret_cast<const char*>(w) + (int64_t)n0 * rowB,
      reinterpret_cast<const char*>(scales) + (int64_t)n0 * sRowB,
      reinterpret_cast<const char*>(biases) + (int64_t)n0 * sRowB, min(16, N - n0), M, K, src,
      qmv_smem, red);
}

}  // namespace mq
