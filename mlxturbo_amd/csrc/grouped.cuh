// Prefill gather_qmm for thin experts: expert-grouped rows with the weights
// dequantized straight into MFMA B registers.
//
// Reference behaviour: moe_grouped_gemm.qmm_segmented (moe_grouped_gemm.py:
// 913-1066): pairs sorted by expert, each tile belongs to one expert; the
// reference notes that thin segments waste tile rows (moe_grouped_gemm.py:
// 61-67).  At prefill MoE widths most experts get tens of rows (config 4:
// 16384 pairs over 512 experts, 32 on average), so a tile is mostly weights:
// the shared-LDS wide tile (qmm_wide.cuh) writes 32 KB of dequantized
// weights to LDS per k-step and reads them back from every wave row for only
// 64 x rows, needs 92 KB of LDS (one workgroup per CU) and measured 1.4 TB/s.
//
// CDNA4 design: a workgroup of NWV waves owns (segment of <= 64 rows, 64 NWV
// weight columns); wave w owns columns 64 w .. 64 w + 63 as two 32-column
// blocks.  Per 64-code k-step, lane l (h = l >> 5) loads 32 codes of column
// (l & 31) of each block, k = 32 h .. 32 h + 31 of the step (one 16-byte load
// per block for 4-bit), dequantizes them exactly (mq_common.h) into the B
// operands of four v_mfma_f32_32x32x16 (MFMA ks takes codes 8 ks .. 8 ks + 7
// of the lane's 32; A rows use the same k order).  The x tile (64 rows x 64
// codes, 9 KB) is staged in LDS, double buffered.  The 8-wave tiles (8-bit
// banks above K = 1024) load their weights into registers; the 4-wave tiles
// of 4-bit banks take them through LDS with the buffer loads' LDS form (16
// columns x 64 bytes per instruction, see thin_tile), 50 KB of LDS per
// workgroup, three per CU.  Every column tile of a segment re-reads its x
// tile, and those re-reads cost as much as the weight stream's access shape
// (a load-only probe: 94 us for the gate/up bank's weights, 132 with the x
// tiles of four column tiles), so from registers long K took 8 waves (512
// columns per x tile); the LDS-form stream made 4 waves the faster again
// (gate/up 272 / 241 us zipf / uniform against 285 / 261).  Global
// loads run PS k-steps ahead in registers (two measured best: deeper
// prefetch lowered occupancy and lost 10-15% on the down bank).  32-row
// blocks past the segment's rows skip their MFMAs.  Measured on the
// config-4 banks at 2048 tokens x top-8 (prep included): down (K=512) 201-212
// us with 4 waves against 265-270 for the wide tile; gate/up (K=2048)
// 427-475 with 4 waves against 341-462 for the wide tile, and with 8 waves
// 279 / 222 zipf / uniform against 302 / 253 (one process, eager loops).
#pragma once
#include "qmm_wide.cuh"

namespace mq {

constexpr int kThinBM = 64;

// One tile of the thin kernel: segment seg of the prep tables (up to BM / Mi
// pairs of one expert; pair p contributes rows p*Mi .. p*Mi+Mi-1 and reads x
// batch x_batch(lhs, p, P, B)) x weight columns [64 NWV col, +64 NWV), 64 NWV
// threads.  Segments of out-of-range experts write zeros.  K % 64 == 0,
// B * Mi * K * 2 < 2^31.
// GLU: (w, scales, biases) is the gate bank and (w2, scales2, biases2) the
// up bank of the same shape; the tile owns output columns [32 NWV col,
// +32 NWV), wave w's two 32-column blocks are the gate and the up rows of
// columns 32 w .. 32 w + 31, and out = swiglu_t(T(gate), T(up)): the two
// gathers and the SwiGLU pass, bit for bit, with each x tile read once for
// both banks.
template <int DT, int BITS, int GS, int PS, int NWV, int BM, bool GLU = false>
__device__ __forceinline__ void thin_tile(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint32_t* __restrict__ w2, const uint16_t* __restrict__ scales2,
    const uint16_t* __restrict__ biases2, const int32_t* __restrict__ lhs,
    uint16_t* __restrict__ out, const int32_t* __restrict__ ws, int P, int B, int Mi, int N,
    int K, int E, int seg, int col, int pofs, unsigned char* __restrict__ wsl0,
    unsigned char* __restrict__ wsl1) {
  constexpr int BN = (GLU ? 32 : 64) * NWV, BK = kWideBK, LD = kWideLD, NT = 64 * NWV;
  constexpr int MB = BM / 32;                   // 32-row blocks of the tile
  static_assert(BM == 64 || BM == 128, "64- or 128-row tiles");
  constexpr int XT = BM * 8;                    // 16-byte x pieces per step
  constexpr int XI = XT >= NT ? XT / NT : 1;    // x pieces per thread per step
  constexpr int WB = BITS / 4;                  // 16-byte loads per lane per block per step
  // 4-wave tiles (short K) take 4-bit weights into LDS by the buffer loads'
  // LDS form (DMA), two k-steps (64 bytes) of 16 columns per load
  // instruction, double buffered in wsl0 / wsl1 (NWV x 4 KB each); each lane
  // then reads its 16 bytes of a step.  Config-4 down bank (K=512), one
  // process: 166.7 / 142.9 us zipf / uniform against 170.3 / 148.1 from
  // registers; 8-wave gate/up tiles (K=2048) lost with it (308.4 against
  // 286.7), and 4-wave gate/up tiles with it beat both (272 zipf).
  constexpr bool DMA = BITS == 4 && NWV == 4;
  static_assert(GS >= 32, "a lane's 32 codes lie in one group");
  using T = T16<DT>;
  __shared__ __align__(16) uint16_t As[2][BM * LD];
  __shared__ uint32_t s_xoff[BM];
  __shared__ int s_orow[BM];
  const int n0 = col * BN;
  const int32_t* perm = ws + 1;
  // the tile's pairs: the segment's from pair pofs on, at most BM / Mi
  const int st0 = perm[P + seg] + pofs, len = min(perm[2 * P + seg] - pofs, BM / Mi);
  if (len <= 0) return;                         // uniform: an empty half of a segment
  const int e = __builtin_amdgcn_readfirstlane(perm[3 * P + seg]);
  const bool valid = e < E;                     // uniform
  const int rows = len * Mi;                    // <= BM
  const int t = threadIdx.x;
  const int ncols = min(BN, N - n0);
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int h = lane >> 5, lr = lane & 31;
  const int G = K / GS, nk = K / BK;
  const int64_t Kw = (int64_t)K * BITS / 32;    // words per weight row
  const int64_t wrow = (int64_t)(valid ? e : 0) * N + n0;
  // columns past ncols are past these ranges and read zeros (never stored)
  __amdgpu_buffer_rsrc_t rw[2], rs[2], rb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const bool up = GLU && j == 1;
    rw[j] = wide_rsrc((up ? w2 : w) + wrow * Kw, (int64_t)ncols * Kw * 4);
    rs[j] = wide_rsrc((up ? scales2 : scales) + wrow * G, (int64_t)ncols * G * 2);
    rb[j] = wide_rsrc((up ? biases2 : biases) + wrow * G, (int64_t)ncols * G * 2);
  }
  const auto xr = wide_rsrc(x, (int64_t)B * Mi * K * 2);
  uint32_t wo[2], so[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = GLU ? 32 * wave + lr : 64 * wave + 32 * j + lr;
    wo[j] = (uint32_t)(c * Kw * 4) + (uint32_t)h * 16u * WB;
    so[j] = (uint32_t)c * (uint32_t)G * 2u;
  }
  // DMA: instruction q of a two-step group covers wave columns 16 q .. 16 q
  // + 15 (block q / 2), four lanes per column; column c's 64 bytes land at
  // LDS c * 64 with their 16-byte pieces permuted by dsw(c), so the per-step
  // reads of 16 (or 8) lanes at consecutive columns hit distinct banks.  A
  // group past the last one reads past the buffer range (zeros, no traffic).
  auto dsw = [](int c) { return ((c >> 1) ^ (c >> 3)) & 3; };
  uint32_t dmo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = 16 * q + (lane >> 2);
    const int cr = GLU ? 32 * wave + (c & 31) : 64 * wave + c;
    dmo[q] = (uint32_t)(cr * Kw * 4) + 16u * (uint32_t)((lane & 3) ^ dsw(c));
  }
  const int ngr = (nk + 1) / 2;                 // two-step groups
  auto wdma = [&](int g, auto slotc) {
    if constexpr (DMA) {
      typedef __attribute__((address_space(3))) void lds_void;
      unsigned char* base = (decltype(slotc)::value == 0 ? wsl0 : wsl1) + wave * 4096;
      const uint32_t go = g < ngr ? (uint32_t)g * 64u : 0x80000000u;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw[q >> 1], (lds_void*)(base + 1024 * q), 16,
                                                 dmo[q], go, 0, 0);
    }
  };
  // x: thread t stages rows (t >> 3) + (NT / 8) i, codes 8 (t & 7) .. +8 of
  // the step (offsets known once the segment's rows are in LDS)
  uint32_t xo[XI];
  int xl[XI];
  struct Stage {
    u32x4 xa[XI];
    u32x4 wv[2][WB];
    uint16_t s[2], b[2];
  };
  // Scales and biases in 16-byte blocks of 8 groups, one load per block,
  // when K / GS is a multiple of 8 and the arrays are 16-byte aligned (the
  // scheme and its measurements are those of wide_tile's FRESH tiles): the
  // loop below is unrolled over a block so each block load and group index
  // is a compile-time position.
  constexpr int SPB = GS / 8;                   // 64-code steps per block
  constexpr bool SBLK = SPB >= PS && SPB <= 8 && SPB % PS == 0;
  const bool sblk = SBLK && G % 8 == 0 && nk % SPB == 0 &&
                    ((uintptr_t)scales | (uintptr_t)biases) % 16 == 0;
  u32x4 ns[2], nb[2], cs[2], cb[2];
  auto bload = [&](int kt) {
    const uint32_t bo = 16u * (uint32_t)(kt * BK / GS / 8);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      ns[j] = __builtin_amdgcn_raw_buffer_load_b128(rs[j], so[j] + bo, 0, 0);
      nb[j] = __builtin_amdgcn_raw_buffer_load_b128(rb[j], so[j] + bo, 0, 0);
    }
  };
  auto xload = [&](Stage& st, int kt) {
#pragma unroll
    for (int i = 0; i < XI; ++i)
      st.xa[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, xo[i], kt * BK * 2, 0);
  };
  // per_step: also load this step's scale and bias (no block path)
  auto wload = [&](Stage& st, int kt, bool per_step) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (!DMA) {
#pragma unroll
        for (int q = 0; q < WB; ++q)
          st.wv[j][q] = __builtin_amdgcn_raw_buffer_load_b128(rw[j], wo[j] + 16u * q,
                                                              k0 * BITS / 8, 0);
      }
      if (per_step) {
        const uint32_t go = so[j] + 2u * (uint32_t)((k0 + 32 * h) / GS);
        st.s[j] = __builtin_amdgcn_raw_buffer_load_b16(rs[j], go, 0, 0);
        st.b[j] = __builtin_amdgcn_raw_buffer_load_b16(rb[j], go, 0, 0);
      }
    }
  };
  auto gload = [&](Stage& st, int kt, bool per_step) {
    xload(st, kt);
    wload(st, kt, per_step);
  };
  auto store_x = [&](const Stage& st, int buf) {
    if (XT >= NT || t < XT) {
#pragma unroll
      for (int i = 0; i < XI; ++i) *reinterpret_cast<u32x4*>(&As[buf][xl[i]]) = st.xa[i];
    }
  };

  // The weights of the first PS steps depend on the expert only: they are
  // issued before the segment's x rows are looked up (xsetup: two more
  // dependent reads and a barrier), inside each prologue branch so that no
  // stage is live across a join (4 waves keep three waves per SIMD).
  // Gate/up zipf 261.7 -> 253.3 us, uniform 229.0 -> 219.7; down 148 -> 145
  // (one process).
  Stage S[PS];
  // the segment's x rows into LDS; false (zeros written) for an invalid expert
  auto xsetup = [&]() -> bool {
    if (t < BM) {
      if (t < rows) {
        const int p = perm[st0 + t / Mi], mi = t % Mi;
        const int xb = x_batch(lhs, p, P, B);
        s_xoff[t] = (uint32_t)(((int64_t)xb * Mi + mi) * K * 2);
        s_orow[t] = p * Mi + mi;
      } else {
        s_xoff[t] = 0xffffffffu;
        s_orow[t] = -1;
      }
    }
    __syncthreads();
    if (!valid) {
      for (int i = t; i < rows * ncols; i += NT) {
        const int r = i / ncols, c = i - r * ncols;
        out[(int64_t)s_orow[r] * N + n0 + c] = 0;
      }
      return false;
    }
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int r = min((t >> 3) + (NT / 8) * i, BM - 1);   // threads past XT: no piece
      const uint32_t ro = (XT >= NT || t < XT) ? s_xoff[r] : 0xffffffffu;
      xo[i] = ro == 0xffffffffu ? 0xffffffffu : ro + 16u * (t & 7);
      xl[i] = r * LD + 8 * (t & 7);
    }
    return true;
  };

  f32x16 acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;
  const int live = rows > 32 ? (rows + 31) / 32 : 1;   // 32-row blocks holding rows

  // One k-step: dequantize codes 8 ks .. 8 ks + 7 of the lane's 32 (B of MFMA
  // ks, per 32-column block) and multiply with the x rows in LDS buffer buf.
  // LB >= 0: step LB of an aligned block, scales from cs / cb
  // DS: with DMA, 2 slot + step of the group (the weights' LDS copy)
  auto step = [&](const Stage& st, int buf, auto lbc, auto dsc) {
    constexpr int LB = decltype(lbc)::value;
    constexpr int DS = decltype(dsc)::value;
    u32x4 wq[2];
    if constexpr (DMA) {
      const unsigned char* base = (DS >> 1 ? wsl1 : wsl0) + wave * 4096;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = 32 * j + lr;
        wq[j] = *reinterpret_cast<const u32x4*>(base + 64 * c + 16 * ((2 * (DS & 1) + h) ^ dsw(c)));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) wq[j] = st.wv[j][0];
    }
    GroupScale g[2];
    bool big = false;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint16_t s16 = st.s[j], b16 = st.b[j];
      if constexpr (LB >= 0) {
        const int e = GS >= BK ? LB * BK / GS % 8 : (LB * BK + 32 * h) / GS % 8;
        const uint32_t w1 = (e & 4) ? ((e & 2) ? cs[j][3] : cs[j][2]) : ((e & 2) ? cs[j][1] : cs[j][0]);
        const uint32_t w2 = (e & 4) ? ((e & 2) ? cb[j][3] : cb[j][2]) : ((e & 2) ? cb[j][1] : cb[j][0]);
        s16 = (uint16_t)((e & 1) ? w1 >> 16 : w1);
        b16 = (uint16_t)((e & 1) ? w2 >> 16 : w2);
      }
      g[j] = make_group(T::to_f32(s16), T::to_f32(b16));
      big |= needs_plain(g[j].s);
    }
    const bool plain = __builtin_amdgcn_ballot_w64(big) != 0;
    const uint16_t* A = &As[buf][lr * LD + 32 * h];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 bq[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        uint32_t o[4];
        if constexpr (BITS == 4) {
          if (plain) deq_word_plain<DT, 4>(wq[j][ks], g[j], o);
          else deq4_word<DT>(wq[j][ks], g[j], o);
        } else {
          const u32x4 v = st.wv[j][ks / 2];
          if (plain) {
            deq_word_plain<DT, 8>(v[2 * (ks % 2)], g[j], o);
            deq_word_plain<DT, 8>(v[2 * (ks % 2) + 1], g[j], o + 2);
          } else {
            deq8_word<DT>(v[2 * (ks % 2)], g[j], o);
            deq8_word<DT>(v[2 * (ks % 2) + 1], g[j], o + 2);
          }
        }
        bq[j] = (u32x4){o[0], o[1], o[2], o[3]};
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
        if (i == 0 || i < live) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(A + 32 * i * LD + 8 * ks);
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<DT>(a, bq[j], acc[i][j]);
        }
    }
  };

  if (sblk) {
    if constexpr (SBLK) {
      if (valid) {
#pragma unroll
        for (int i = 0; i < PS; ++i) wload(S[i], i, false);
        wdma(0, std::integral_constant<int, 0>{});
        wdma(1, std::integral_constant<int, 1>{});
        bload(0);
      }
      if (!xsetup()) return;
#pragma unroll
      for (int i = 0; i < PS; ++i) xload(S[i], i);
      store_x(S[0], 0);
      __syncthreads();
      // step u of a block: as the loop below, and the block of step kt + SPB
      // is loaded with step kt + SPB's weights (PS steps ahead)
      for (int kt = 0; kt < nk; kt += SPB) {
        static_for<0, SPB>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          if constexpr (u == 0) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              cs[j] = ns[j];
              cb[j] = nb[j];
            }
          }
          step(S[u % PS], u & 1, uc, std::integral_constant<int, 2 * ((u >> 1) & 1) + (u & 1)>{});
          // a group's weights are read: its slot takes the group after next
          if constexpr (u & 1) wdma(((kt + u) >> 1) + 2, std::integral_constant<int, (u >> 1) & 1>{});
          gload(S[u % PS], min(kt + u + PS, nk - 1), false);
          if constexpr (u + PS == SPB) bload(min(kt + SPB, nk - SPB));
          store_x(S[(u + 1) % PS], (u + 1) & 1);
          __syncthreads();
        });
      }
    }
  } else {
    if (valid) {
#pragma unroll
      for (int i = 0; i < PS; ++i) wload(S[i], min(i, nk - 1), true);
      wdma(0, std::integral_constant<int, 0>{});
      wdma(1, std::integral_constant<int, 1>{});
    }
    if (!xsetup()) return;
#pragma unroll
    for (int i = 0; i < PS; ++i) xload(S[i], min(i, nk - 1));
    store_x(S[0], 0);
    __syncthreads();
    // At step k: LDS buffer k & 1 holds x of step k; S[k % PS] holds step k's
    // weights (with DMA: its scales; the weights are in slot (k / 2) & 1) and
    // is reloaded with step k + PS once they are multiplied; S[(k + i) % PS]
    // holds step k + i.  The body is unrolled over lcm(PS, 2) steps (4 with
    // DMA) so stage, buffer and slot indices are constants; the last steps
    // reload step nk - 1 (valid memory, unused), so the loads need no
    // conditions.
    constexpr int U = DMA ? 4 : PS % 2 ? 2 * PS : PS;
    static_assert(U % PS == 0, "whole stage rounds per body");
    for (int kt = 0; kt < nk; kt += U) {
      static_for<0, U>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if (u == 0 || kt + u < nk) {                // uniform
          step(S[u % PS], u & 1, std::integral_constant<int, -1>{},
               std::integral_constant<int, 2 * ((u >> 1) & 1) + (u & 1)>{});
          if constexpr (u & 1) wdma(((kt + u) >> 1) + 2, std::integral_constant<int, (u >> 1) & 1>{});
          gload(S[u % PS], min(kt + u + PS, nk - 1), true);
          store_x(S[(u + 1) % PS], (u + 1) & 1);
          __syncthreads();
        }
      });
    }
  }

  // the last groups' loads (past the range, zeros) may still be landing in
  // LDS: none may be in flight when the workgroup's LDS is given back
  if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0);
  // D[row][col] of a 32x32 tile: col = lane & 31, row = 8*(e/4) + 4*(lane>>5) + e%4
  if constexpr (GLU) {
    const int c = 32 * wave + lr;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int r = 32 * i + 8 * (q >> 2) + 4 * h + (q & 3);
        if (r < rows && c < ncols)
          out[(int64_t)s_orow[r] * N + n0 + c] =
              swiglu_t<DT>(T::round1(acc[i][0][q]), T::round1(acc[i][1][q]));
      }
  } else {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = 64 * wave + 32 * j + lr;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int r = 32 * i + 8 * (q >> 2) + 4 * h + (q & 3);
          if (r < rows && c < ncols) out[(int64_t)s_orow[r] * N + n0 + c] = T::round1(acc[i][j][q]);
        }
      }
  }
}

// 1-D grid, 64 NWV threads, tiles placed by grouped_tile.  CLS2 false: the
// tiles of the prep tables' size class cls (segments of up to 64 / Mi pairs),
// ceil(N / (64 NWV)) x its segment bound workgroups.  CLS2 true: class 1
// (segments of up to 2 (64 / Mi) pairs, 128-row tiles) in the first 8 q1
// workgroups (q1 = its tiles / 8, rounded up), then class 0 (64-row tiles);
// cls is ignored.  Each height runs its own code (a 128-row body for every
// tile made the 64-row ones slower).  HALVES: class 1's segments run as two
// 64-row tiles each (first and second 64 / Mi pairs, adjacent tiles), the
// work of one-class tables, from the same two-class tables.
template <int DT, int BITS, int GS, int PS, int NWV, bool CLS2, bool HALVES = false,
          bool GLU = false>
__global__ __launch_bounds__(64 * NWV) void qmm_grouped_thin_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint32_t* __restrict__ w2, const uint16_t* __restrict__ scales2,
    const uint16_t* __restrict__ biases2, const int32_t* __restrict__ lhs,
    uint16_t* __restrict__ out, const int32_t* __restrict__ ws, int P, int B, int Mi, int N,
    int K, int E, int cls) {
  // the 4-wave 4-bit tiles' weight slots (thin_tile's DMA), shared by both
  // heights
  constexpr int WSL = BITS == 4 && NWV == 4 ? NWV * 4096 : 16;
  __shared__ __align__(16) unsigned char wsl0[WSL];
  __shared__ __align__(16) unsigned char wsl1[WSL];
  const int32_t* hdr = ws + gather_ws_header(P);
  constexpr int BN = (GLU ? 32 : 64) * NWV;     // output columns per tile
  const int ncol = (N + BN - 1) / BN;
  int bi = blockIdx.x;
  constexpr int H1 = HALVES ? 2 : 1;           // tiles per class-1 segment
  if constexpr (CLS2) {
    cls = 1;
    const int q1 = (H1 * (hdr[2] - hdr[1]) * ncol + 7) / 8;
    if (bi >= 8 * q1) {
      bi -= 8 * q1;
      cls = 0;
    }
  }
  const int s0 = hdr[2 - cls];
  const int nv = (hdr[3 - cls] - s0) * (CLS2 && cls == 1 ? H1 : 1);
  int seg, col;
  if (!grouped_tile(bi, nv, ncol, seg, col)) return;
  if (CLS2 && cls == 1 && !HALVES)
    thin_tile<DT, BITS, GS, PS, NWV, 128, GLU>(x, w, scales, biases, w2, scales2, biases2, lhs,
                                                out, ws, P, B, Mi, N, K, E, seg + s0, col, 0, wsl0, wsl1);
  else if (CLS2 && cls == 1)
    thin_tile<DT, BITS, GS, PS, NWV, 64, GLU>(x, w, scales, biases, w2, scales2, biases2, lhs,
                                               out, ws, P, B, Mi, N, K, E, (seg >> 1) + s0, col,
                                               (seg & 1) * (64 / Mi), wsl0, wsl1);
  else
    thin_tile<DT, BITS, GS, PS, NWV, 64, GLU>(x, w, scales, biases, w2, scales2, biases2, lhs,
                                               out, ws, P, B, Mi, N, K, E, seg + s0, col, 0, wsl0, wsl1);
}

}  // namespace mq
