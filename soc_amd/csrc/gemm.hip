// gemm.hip - prefill projections C = A . W^T with fp16 weights, on MFMA: from fp32 activations (register-staged
// split into hi/lo fp16 parts) or from fp16 activations written by their producers (direct-to-LDS pipeline).
//
// Reference computation: Linear::Forward over T rows (Mac/cpu/src/linear.cpp:145-157), fp32 accumulation.
#include "kernels.h"

namespace soc {

// ------------------------------------------------------------------------------------------------------------
// MFMA GEMM: BM x 128 output tile per 256-thread block (BM = 128, or 64 when 128-row tiles would leave CUs idle),
// K slices of 32 staged in LDS (double buffered), each wave owns a (BM / 2) x 64 quadrant as tiles of
// v_mfma_f32_32x32x16_f16. Activations arrive in fp32 and are split on the way into LDS into hi = f16(a) and
// lo = f16((a - hi) * 2^11); with SPLIT the product is hi.W + 2^-11 lo.W, which keeps about 22 bits of each
// activation (weights are exact fp16), so the result tracks the fp32 reference.
// Global loads run two K slices ahead of the MFMAs (two register stages), so a slice's loads have two slices of
// MFMA work to arrive in.
// EPI_SWIGLU stages 64 gate rows and the matching 64 up rows per tile; a wave holds gate and up accumulators of the
// same outputs in the same registers and writes silu(g) * u.
// ------------------------------------------------------------------------------------------------------------
namespace {
constexpr int MBN = 128, MBK = 32, MPAD = 8;  // LDS rows padded to 40 halves (80 B)
constexpr int MLD = MBK + MPAD;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
}  // namespace

template <int EPI, bool SPLIT, int BM>
__global__ __launch_bounds__(256, 2) void k_gemm_mfma(GemmArgs g) {
  constexpr int NA = SPLIT ? 2 : 1;
  constexpr int MI = BM / 64;         // 32-row MFMA tiles per wave
  constexpr int AV = BM * MBK / 1024;  // float4 of A per thread per slice
  __shared__ _Float16 As[2][NA][BM * MLD];
  __shared__ _Float16 Bs[2][MBN * MLD];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  // XCD-aware tile order: blocks are dispatched round-robin over the 8 XCDs, so block b runs on XCD b % 8. Each
  // XCD takes a contiguous eighth of the column tiles (its weight rows stay in its L2) and walks them fastest, so
  // its co-resident blocks share activation row tiles too.
  const int mt = (g.M + BM - 1) / BM, nt = gridDim.x / mt;
  int mtile, ntile;
  if (nt % 8 == 0) {
    const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3, per = nt >> 3;
    ntile = xcd * per + j % per;
    mtile = j / per;
  } else {
    ntile = blockIdx.x % nt;
    mtile = blockIdx.x / nt;
  }
  const int m0 = mtile * BM;
  // output columns covered by this block: plain GEMM 128, SwiGLU 64 (gate/up pairs)
  const int n0 = ntile * (EPI == EPI_SWIGLU ? MBN / 2 : MBN);

  // global -> register staging (two stages): A BM x 32 fp32, W 128 x 32 fp16 = 512 x 16 B (2 per thread)
  f32x4 ra[2][AV];
  u32x4 rb[2][2];
  auto load_tiles = [&](int st, int k0) {
#pragma unroll
    for (int e = 0; e < AV; ++e) {
      const int idx = tid + e * 256;
      const int r = idx >> 3, c = (idx & 7) * 4;
      const int m = m0 + r;
      ra[st][e] = (m < g.M) ? *reinterpret_cast<const f32x4*>(g.a + static_cast<size_t>(m) * g.lda + k0 + c)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int idx = tid + e * 256;
      const int r = idx >> 2, c = (idx & 3) * 8;
      const f16* src;
      int n;
      if constexpr (EPI == EPI_SWIGLU) {
        n = n0 + (r & 63);
        src = r < 64 ? g.w : g.w2;
      } else {
        n = n0 + r;
        src = g.w;
      }
      rb[st][e] = (n < g.N) ? load16(src + static_cast<size_t>(n) * g.K + k0 + c) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_tiles = [&](int st, int buf) {
#pragma unroll
    for (int e = 0; e < AV; ++e) {
      const int idx = tid + e * 256;
      const int r = idx >> 3, c = (idx & 7) * 4;
      f16x4 hi, lo;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = ra[st][e][i];
        const _Float16 h = static_cast<_Float16>(v);
        hi[i] = h;
        lo[i] = static_cast<_Float16>((v - static_cast<float>(h)) * 2048.0f);
      }
      *reinterpret_cast<f16x4*>(&As[buf][0][r * MLD + c]) = hi;
      if constexpr (SPLIT) *reinterpret_cast<f16x4*>(&As[buf][NA - 1][r * MLD + c]) = lo;
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int idx = tid + e * 256;
      const int r = idx >> 2, c = (idx & 3) * 8;
      *reinterpret_cast<u32x4*>(&Bs[buf][r * MLD + c]) = rb[st][e];
    }
  };

  f32x16 acc[MI][2], acc_lo[MI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
        acc_lo[i][j][r] = 0.0f;
      }

  // B sub-tile rows of this wave: plain = wn*64 + t*32; SwiGLU: t = 0 gate rows wn*32, t = 1 up rows 64 + wn*32
  const int brow[2] = {EPI == EPI_SWIGLU ? wn * 32 : wn * 64, EPI == EPI_SWIGLU ? 64 + wn * 32 : wn * 64 + 32};
  const int KT = g.K / MBK;
  // slice kt is loaded into register stage kt & 1 and stored into LDS buffer kt & 1
  load_tiles(0, 0);
  if (KT > 1) load_tiles(1, MBK);
  store_tiles(0, 0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 2 < KT) load_tiles(buf, (kt + 2) * MBK);  // stage buf held slice kt, already in LDS
#pragma unroll
    for (int ks = 0; ks < MBK / 16; ++ks) {
      const int kc = ks * 16 + (lane >> 5) * 8;
      h8 bf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        bf[t] = *reinterpret_cast<const h8*>(&Bs[buf][(brow[t] + (lane & 31)) * MLD + kc]);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int arow = wm * (BM / 2) + i * 32 + (lane & 31);
        const h8 ah = *reinterpret_cast<const h8*>(&As[buf][0][arow * MLD + kc]);
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bf[t], acc[i][t], 0, 0, 0);
        if constexpr (SPLIT) {
          const h8 al = *reinterpret_cast<const h8*>(&As[buf][NA - 1][arow * MLD + kc]);
#pragma unroll
          for (int t = 0; t < 2; ++t)
            acc_lo[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bf[t], acc_lo[i][t], 0, 0, 0);
        }
      }
    }
    if (kt + 1 < KT) store_tiles(buf ^ 1, buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds D[m][n] for n = lane % 32, m = (r / 4) * 8 + (lane / 32) * 4 + r % 4
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (m >= g.M) continue;
      float v[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) v[t] = acc[i][t][r] + (SPLIT ? acc_lo[i][t][r] * (1.0f / 2048.0f) : 0.0f);
      if constexpr (EPI == EPI_SWIGLU) {
        const int n = n0 + wn * 32 + (lane & 31);
        if (n < g.N) g.c[static_cast<size_t>(m) * g.ldc + n] = silu_ref(v[0]) * v[1];
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int n = n0 + wn * 64 + t * 32 + (lane & 31);
          if (n < g.N) {
            float* dst = g.c + static_cast<size_t>(m) * g.ldc + n;
            *dst = EPI == EPI_RESIDUAL ? *dst + v[t] : v[t];
          }
        }
      }
    }
}

// ------------------------------------------------------------------------------------------------------------
// MFMA GEMM on pre-split activations: A arrives as hi and lo fp16 arrays (written by the producing kernel with the
// same split as above), so no register staging is needed and all three operands go global -> LDS with
// global_load_lds_dwordx4 (16 bytes per lane into 1 KB of LDS per wave instruction) through an ST-slot ring of
// BK-deep K slices. A slot is refilled (slice kt + ST) by the barrier that follows the last LDS read of slice kt,
// so ST slices are in flight while a slice's last 16-deep step runs; before that barrier a wave waits only for its
// own loads of slice kt + 1 (vmcnt) and for its LDS reads (lgkmcnt). The MFMA operands of the next 16-deep step are
// read from LDS while the current step's MFMAs run (two register sets used in turn), one read issued after each
// MFMA. Rows are BK halves with the 16-byte chunk c of row r stored at slot c ^ ((r >> 2) & 3) (BK = 32) or
// c ^ ((r >> 1) & 7) (BK = 64): the 16 rows a b128 read phase touches land on different bank groups.
// BM x BN tile per block of NWM x NWN waves (each a (BM/NWM) x (BN/NWN) part, v_mfma_f32_32x32x16_f16; every
// configuration accumulates the same 16-deep MFMA steps in the same K order). Tiles are dealt to the
// eight XCDs as an mx x (8 / mx) grid of rectangles (block b runs on XCD b % 8), mx chosen to minimise the bytes
// of A and W each XCD's L2 has to fetch. The products and their order match k_gemm_mfma<EPI, true, .> exactly, or
// with LO = false (single fp16 activations, no lo part) those of k_gemm_mfma<EPI, false, .>.
// EPI_SWIGLU with ch/cl set writes silu(g) * u as the hi/lo pair the down projection consumes.
// ------------------------------------------------------------------------------------------------------------
namespace {
// LDS has 64 banks of 4 bytes, and a 16-byte read serves 16 lanes per cycle: the 16 rows one read phase touches
// (lanes 0-15, 16-31, ...) must hit 16 different 16-byte bank groups. A 64-half row is half a bank row, so rows r and
// r + 1 sit in different halves and the slot must differ between rows of equal parity: c ^ ((r >> 1) & 7). A
// 32-half row is a quarter: c ^ ((r >> 2) & 3).
template <int BK>
__device__ __forceinline__ int chunk_slot(int r, int c) {
  if constexpr (BK == 32) return c ^ ((r >> 2) & 3);
  else return c ^ ((r >> 1) & 7);
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  // vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt not waited on
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// wait until at most n slices (of IPT loads each) issued after the awaited one are in flight, n <= MAXN
template <int IPT, int MAXN>
__device__ __forceinline__ void wait_slices(int n) {
  if constexpr (MAXN <= 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= MAXN) wait_vmcnt<MAXN * IPT>();
    else wait_slices<IPT, MAXN - 1>(n);
  }
}
// a barrier with no fence (a fenced one would also wait for the loads of later slices still in flight); the
// signal fences keep the compiler from moving LDS accesses across it
__device__ __forceinline__ void block_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
}  // namespace

template <int EPI, int BM, int BN, int ST, int MINB, int BK, bool LO, int NWM, int NWN>
__global__ __launch_bounds__(64 * NWM * NWN, MINB) void k_gemm_split(GemmSplitArgs g, int mx) {
  constexpr int NW = NWM * NWN;                    // waves: NWM x NWN, each a WTM x WTN part of the tile
  constexpr int WTM = BM / NWM, WTN = BN / NWN;
  constexpr int MI = WTM / 32, NJ = WTN / 32;      // 32x32 MFMA tiles per wave
  constexpr int RPI = 1024 / (BK * 2);             // rows per 1 KB wave instruction
  constexpr int CPR = BK / 8;                      // 16-byte chunks per row
  constexpr int AP = LO ? 2 : 1;                   // activation parts: hi and lo, or hi alone
  constexpr int AI = BM / RPI / NW, WI = BN / RPI / NW;  // DMA instructions per wave per slice: each A part, W
  constexpr int IPT = AP * AI + WI;
  constexpr int KS = BK / 16;  // 16-deep MFMA steps per slice
  constexpr int STAGE_H = (AP * BM + BN) * BK;
  static_assert(EPI != EPI_SWIGLU || NJ % 2 == 0, "SwiGLU pairs gate and up tiles within a wave");
  static_assert(KS % 2 == 0 && ST >= 2 && AI >= 1 && WI >= 1, "tile shape");
  static_assert(AI * RPI * NW == BM && WI * RPI * NW == BN && MI >= 1 && NJ >= 1, "tile shape");
  extern __shared__ __attribute__((aligned(16))) _Float16 slds[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / NWN, wn = wid % NWN;
  const int mt = (g.M + BM - 1) / BM, nt = gridDim.x / mt;
  int mtile, ntile;
  if (mx > 0) {  // XCD rectangle (b % 8) of (mt / mx) x (nt / nx) tiles, walked along N
    const int nx = 8 / mx, grp = blockIdx.x & 7, j = blockIdx.x >> 3;
    const int tm = mt / mx, tn = nt / nx;
    mtile = (grp / nx) * tm + j / tn;
    ntile = (grp % nx) * tn + j % tn;
  } else {
    ntile = blockIdx.x % nt;
    mtile = blockIdx.x / nt;
  }
  const int m0 = mtile * BM;
  const int n0 = ntile * (EPI == EPI_SWIGLU ? BN / 2 : BN);
  const int KT = g.K / BK;
  auto issue = [&](int kt, int st) {
    _Float16* base = slds + st * STAGE_H;
    const int k0 = kt * BK;
#pragma unroll
    for (int h = 0; h < AI; ++h) {
      const int rb = (wid * AI + h) * RPI;
      const int r = rb + lane / CPR;
      const int c = chunk_slot<BK>(r, lane % CPR);
      const size_t off = static_cast<size_t>(min(m0 + r, g.M - 1)) * g.lda + k0 + c * 8;
      __builtin_amdgcn_global_load_lds(g.ah + off, base + rb * BK, 16, 0, 0);
      if constexpr (LO) __builtin_amdgcn_global_load_lds(g.al + off, base + BM * BK + rb * BK, 16, 0, 0);
    }
#pragma unroll
    for (int h = 0; h < WI; ++h) {
      const int rb = (wid * WI + h) * RPI;
      const int r = rb + lane / CPR;
      const int c = chunk_slot<BK>(r, lane % CPR);
      int n;
      const f16* src;
      if constexpr (EPI == EPI_SWIGLU) {
        n = n0 + (r % (BN / 2));
        src = r < BN / 2 ? g.w : g.w2;
      } else {
        n = n0 + r;
        src = g.w;
      }
      n = min(n, g.N - 1);
      __builtin_amdgcn_global_load_lds(src + static_cast<size_t>(n) * g.K + k0 + c * 8, base + AP * BM * BK + rb * BK,
                                       16, 0, 0);
    }
  };

  f32x16 acc[MI][NJ], acc_lo[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
        acc_lo[i][j][r] = 0.0f;
      }
  // W rows of the wave's 32-column tiles: plain wn*WTN + t*32; SwiGLU: gate rows wn*WTN/2 + t*32 (t < NJ/2), the
  // matching up rows BN/2 + the same
  int brow[NJ];
#pragma unroll
  for (int t = 0; t < NJ; ++t)
    brow[t] = EPI == EPI_SWIGLU ? (t / (NJ / 2)) * (BN / 2) + wn * (WTN / 2) + (t % (NJ / 2)) * 32 : wn * WTN + t * 32;

  h8 a0[MI][2], b0[NJ], a1[MI][2], b1[NJ];  // the two operand sets
  auto read = [&](h8 (&fa)[MI][2], h8 (&fb)[NJ], int st, int ks) {
    const _Float16* Ah = slds + st * STAGE_H;
    const _Float16* Al = Ah + BM * BK;
    const _Float16* Ws = Ah + AP * BM * BK;
    const int c = 2 * ks + (lane >> 5);
#pragma unroll
    for (int t = 0; t < NJ; ++t) {
      const int r = brow[t] + (lane & 31);
      fb[t] = *reinterpret_cast<const h8*>(Ws + r * BK + chunk_slot<BK>(r, c) * 8);
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int r = wm * WTM + i * 32 + (lane & 31);
      const int off = r * BK + chunk_slot<BK>(r, c) * 8;
      fa[i][0] = *reinterpret_cast<const h8*>(Ah + off);
      if constexpr (LO) fa[i][1] = *reinterpret_cast<const h8*>(Al + off);
    }
  };
  auto mma = [&](const h8 (&fa)[MI][2], const h8 (&fb)[NJ]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int t = 0; t < NJ; ++t) {
        acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i][0], fb[t], acc[i][t], 0, 0, 0);
        if constexpr (LO)
          acc_lo[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i][1], fb[t], acc_lo[i][t], 0, 0, 0);
      }
  };
  // one MFMA, one LDS read, ... then the remaining MFMAs
  auto interleave = [&]() {
    constexpr int NR = AP * MI + NJ, NM = AP * MI * NJ;  // LDS operand reads and MFMAs per 16-deep step
    constexpr int NP = NR < NM ? NR : NM;
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (NM > NP) __builtin_amdgcn_sched_group_barrier(0x008, NM - NP, 0);
    if constexpr (NR > NP) __builtin_amdgcn_sched_group_barrier(0x100, NR - NP, 0);
  };

#pragma unroll
  for (int p = 0; p < ST; ++p)
    if (p < KT) issue(p, p);
  wait_slices<IPT, ST - 1>(KT - 1);
  block_barrier();
  read(a0, b0, 0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    const int st = kt % ST;
#pragma unroll
    for (int ks = 0; ks < KS; ks += 2) {
      // the first half of each step pair at raised priority: the waves of a SIMD fall into alternating phases, one
      // issuing its MFMAs while another reads its next operands (2048-token prefill 5.90 -> 5.79 ms)
      __builtin_amdgcn_s_setprio(1);
      read(a1, b1, st, ks + 1);
      mma(a0, b0);
      interleave();
      __builtin_amdgcn_s_setprio(0);
      if (ks + 2 < KS) {
        read(a0, b0, st, ks + 2);
        mma(a1, b1);
        interleave();
      } else {
        if (kt + 1 < KT) {
          wait_slices<IPT, ST - 2>(KT - 2 - kt);  // own loads of slice kt + 1 landed
          wait_lgkmcnt0();                         // own reads of slot st done
          block_barrier();
          if (kt + ST < KT) issue(kt + ST, st);
          read(a0, b0, (kt + 1) % ST, 0);
        }
        mma(a1, b1);
      }
    }
  }
  // epilogue: lane holds D[m][n] for n = lane % 32, m = (r / 4) * 8 + (lane / 32) * 4 + r % 4
  if constexpr (EPI == EPI_QKV) {
    // the tile's 128 columns are one head: park the tile in LDS, then each wave takes BM / NW of its rows with lane l
    // holding dims (l, l + 64), as the q/k-norm kernel does, so q, k and v come out bit-identical to it
    static_assert(BN == 128, "one 128-dim head per tile");
    static_assert(static_cast<size_t>(BM) * (BN + 1) * 4 <= static_cast<size_t>(ST) * STAGE_H * 2, "park area");
    constexpr int LDX = BN + 1;
    float* xs = reinterpret_cast<float*>(slds);
    __syncthreads();  // every wave's MFMA operand reads of the ring are done
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
#pragma unroll
        for (int t = 0; t < NJ; ++t)
          xs[ml * LDX + wn * WTN + t * 32 + (lane & 31)] =
              LO ? acc[i][t][r] + acc_lo[i][t][r] * (1.0f / 2048.0f) : acc[i][t][r];
      }
    __syncthreads();
    const GemmSplitArgs::Qkv& q = g.qkv;
    const int head = n0 / BN;  // q heads, then k heads, then v heads
    const bool rope = head < q.nq + q.nkv;
    // every load of the wave's BM / NW rows (values from LDS, the head's gains, the rows' RoPE table entries) is
    // issued before the first store, so none of them waits behind a store it might alias
    constexpr int RW = BM / NW;
    float x0[RW], x1[RW], cr[RW], sr[RW];
    float g0 = 1.0f, g1 = 1.0f;
    if (rope) {
      const f16* gn = head < q.nq ? q.q_gain : q.k_gain;
      g0 = static_cast<float>(ld_global(gn, lane));
      g1 = static_cast<float>(ld_global(gn, lane + 64));
    }
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
      const int ml = wid * RW + rr;
      x0[rr] = xs[ml * LDX + lane];
      x1[rr] = xs[ml * LDX + lane + 64];
      cr[rr] = sr[rr] = 0.0f;
      if (rope) {
        const int pos = q.pos_base + min(m0 + ml, g.M - 1);
        cr[rr] = q.rope_cos[static_cast<size_t>(pos) * 64 + lane];
        sr[rr] = q.rope_sin[static_cast<size_t>(pos) * 64 + lane];
      }
    }
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
      const int m = m0 + wid * RW + rr;
      if (m >= g.M) break;  // wave-uniform
      const int pos = q.pos_base + m;
      if (rope) norm_rope_pair(x0[rr], x1[rr], g0, g1, q.eps, cr[rr], sr[rr]);
      if (head < q.nq) {
        float* dst = q.q_out + static_cast<size_t>(m) * q.nq * 128 + head * 128;
        dst[lane] = x0[rr];
        dst[lane + 64] = x1[rr];
      } else {
        const bool is_k = head < q.nq + q.nkv;
        const int kvh = is_k ? head - q.nq : head - q.nq - q.nkv;
        const size_t base = static_cast<size_t>(q.slot) * q.slot_stride + static_cast<size_t>(q.layer) * q.layer_stride +
                            (static_cast<size_t>(kvh) * q.cap + pos) * 128;
        f16* cache = is_k ? q.kcache : q.vcache;
        cache[base + lane] = static_cast<f16>(x0[rr]);
        cache[base + lane + 64] = static_cast<f16>(x1[rr]);
      }
    }
    return;
  }
  // residual: every element of the wave's part of C is read before the first store (otherwise each read waits
  // behind the store before it, which the compiler cannot prove does not alias it)
  float res[EPI == EPI_RESIDUAL ? MI : 1][EPI == EPI_RESIDUAL ? NJ : 1][16];
  if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = min(m0 + wm * WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), g.M - 1);
#pragma unroll
        for (int t = 0; t < NJ; ++t) {
          const int n = min(n0 + wn * WTN + t * 32 + (lane & 31), g.N - 1);
          res[i][t][r] = g.c[static_cast<size_t>(m) * g.ldc + n];
        }
      }
  }
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (m >= g.M) continue;
      float v[NJ];
#pragma unroll
      for (int t = 0; t < NJ; ++t) v[t] = LO ? acc[i][t][r] + acc_lo[i][t][r] * (1.0f / 2048.0f) : acc[i][t][r];
      if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int t = 0; t < NJ / 2; ++t) {
          const int n = n0 + wn * (WTN / 2) + t * 32 + (lane & 31);
          if (n < g.N) {
            const float y = silu_ref(v[t]) * v[t + NJ / 2];
            const size_t o = static_cast<size_t>(m) * g.ldc + n;
            if (g.ch != nullptr) {
              const _Float16 hi = static_cast<_Float16>(y);
              g.ch[o] = hi;
              if (g.cl != nullptr) g.cl[o] = static_cast<_Float16>((y - static_cast<float>(hi)) * 2048.0f);
            } else {
              g.c[o] = y;
            }
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < NJ; ++t) {
          const int n = n0 + wn * WTN + t * 32 + (lane & 31);
          if (n < g.N) g.c[static_cast<size_t>(m) * g.ldc + n] = EPI == EPI_RESIDUAL ? res[i][t][r] + v[t] : v[t];
        }
      }
    }
}

namespace {
// mx for the XCD rectangles: the split of the mt x nt tile grid into mx x (8 / mx) parts that minimises the bytes
// of A (4 per element: hi + lo) and W (2 per element) per XCD; 0 (row-major tile order) when none divides evenly.
int xcd_split(int mt, int nt, double abytes, double wbytes) {
  int best = 0;
  double cost = 0.0;
  for (int mx = 1; mx <= 8; mx *= 2) {
    if (mt % mx != 0 || nt % (8 / mx) != 0) continue;
    const double c = abytes / mx + wbytes / (8 / mx);
    if (best == 0 || c < cost) {
      best = mx;
      cost = c;
    }
  }
  return best;
}

template <int EPI, int BM, int BN, int ST, int MINB, int BK, bool LO, int NWM = 2, int NWN = 2>
hipError_t launch_split_cfg(const GemmSplitArgs& g, hipStream_t s) {
  constexpr int AP = LO ? 2 : 1;
  const int bn = EPI == EPI_SWIGLU ? BN / 2 : BN;
  const int mt = (g.M + BM - 1) / BM, nt = (g.N + bn - 1) / bn;
  const int mx = xcd_split(mt, nt, 2.0 * AP * g.M * g.K, 2.0 * (EPI == EPI_SWIGLU ? 2 : 1) * g.N * g.K);
  const size_t lds = static_cast<size_t>(ST) * (AP * BM + BN) * BK * sizeof(_Float16);
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(k_gemm_split<EPI, BM, BN, ST, MINB, BK, LO, NWM, NWN>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((k_gemm_split<EPI, BM, BN, ST, MINB, BK, LO, NWM, NWN>), dim3(mt * nt), dim3(64 * NWM * NWN), lds, s,
                     g, mx);
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_split_epi(const GemmSplitArgs& g, hipStream_t s) {
  // 128-row tiles on 8 waves when they still give every CU its blocks (long prompts; measured on the Qwen3-0.6B
  // prefill at 2048 tokens): a block's 8 waves share twice the rows of A and W per LDS slice, and two such blocks per
  // CU keep 16 waves resident. QKV (hi/lo activations): 128 x 128 tiles, 32-deep slices in a 3-slot ring (56 -> 53
  // us); gate/up: 128 x 128 (64 gate and 64 up rows), 64-deep slices in a 2-slot ring (44 -> 39.5 us); o/down
  // (N <= 1024, one block per CU): 128 x 64, a 4-slot ring (29 -> 28 us).
  const int mt128 = (g.M + 127) / 128;
  if constexpr (EPI == EPI_QKV) {
    if (g.al != nullptr && mt128 * (g.N / 128) >= 512) return launch_split_cfg<EPI, 128, 128, 3, 2, 32, true, 4, 2>(g, s);
  }
  if constexpr (EPI == EPI_SWIGLU) {
    // gate/up of a full chip of 256-row tiles: 256 x 192 (96 gate and 96 up rows) on 8 waves of 32 rows, one block
    // per CU, one tile each (2048 tokens: 39.7 -> 37.9 us; 128 x 128 tiles make 1.5 rounds of two blocks per CU)
    if (g.al == nullptr && g.K % 64 == 0 && ((g.M + 255) / 256) * ((g.N + 95) / 96) >= 256)
      return launch_split_cfg<EPI, 256, 192, 2, 1, 64, false, 8, 1>(g, s);
    if (g.al == nullptr && g.K % 64 == 0 && mt128 * ((g.N + 63) / 64) >= 512)
      return launch_split_cfg<EPI, 128, 128, 2, 2, 64, false, 4, 2>(g, s);
  }
  // 64 x 128 tiles, two blocks per CU: 64-deep slices in a 2-slot ring, or 32-deep ones in a 4-slot ring when K
  // is not a multiple of 64 (measured on the Qwen3-0.6B prefill shapes at 2048 tokens). The residual projections
  // of <= 1024 columns (o and down) would get one 64 x 128 tile per CU; 64 x 64 tiles, up to three blocks per CU,
  // give them twice the blocks (2048 tokens: 8.29 -> 7.97 ms per prefill); on single fp16 activations a 3-slot ring
  // fits three blocks per CU and hides more of the load latency (6.92 -> 6.69 ms)
  if constexpr (EPI == EPI_RESIDUAL) {
    if (g.K % 64 == 0 && g.N <= 1024) {
      if (g.al == nullptr && mt128 * ((g.N + 63) / 64) >= 256)
        return launch_split_cfg<EPI, 128, 64, 4, 1, 64, false, 4, 2>(g, s);
      return g.al != nullptr ? launch_split_cfg<EPI, 64, 64, 2, 3, 64, true>(g, s)
                             : launch_split_cfg<EPI, 64, 64, 3, 3, 64, false>(g, s);
    }
  }
  if (g.al != nullptr)
    return g.K % 64 == 0 ? launch_split_cfg<EPI, 64, 128, 2, 2, 64, true>(g, s)
                         : launch_split_cfg<EPI, 64, 128, 4, 2, 32, true>(g, s);
  return g.K % 64 == 0 ? launch_split_cfg<EPI, 64, 128, 2, 2, 64, false>(g, s)
                       : launch_split_cfg<EPI, 64, 128, 4, 2, 32, false>(g, s);
}
}  // namespace

bool gemm_split_supported(const GemmSplitArgs& g) {
  return g.K % 32 == 0 && g.lda % 8 == 0 && g.M > 0 && g.N > 0 &&
         (reinterpret_cast<uintptr_t>(g.ah) | reinterpret_cast<uintptr_t>(g.al) |
          reinterpret_cast<uintptr_t>(g.w) | reinterpret_cast<uintptr_t>(g.w2)) % 16 == 0;
}

hipError_t launch_gemm_split(const GemmSplitArgs& g, int epi, hipStream_t s) {
  if (!gemm_split_supported(g)) return hipErrorInvalidValue;
  if (epi == EPI_SWIGLU && (g.w2 == nullptr || (g.cl != nullptr && g.ch == nullptr))) return hipErrorInvalidValue;
  if (epi == EPI_QKV && (g.N != (g.qkv.nq + 2 * g.qkv.nkv) * 128 || g.qkv.q_out == nullptr ||
                         g.qkv.kcache == nullptr || g.qkv.vcache == nullptr))
    return hipErrorInvalidValue;
  switch (epi) {
    case EPI_STORE: return launch_split_epi<EPI_STORE>(g, s);
    case EPI_RESIDUAL: return launch_split_epi<EPI_RESIDUAL>(g, s);
    case EPI_SWIGLU: return launch_split_epi<EPI_SWIGLU>(g, s);
    case EPI_QKV: return launch_split_epi<EPI_QKV>(g, s);
    default: return hipErrorInvalidValue;
  }
}

bool gemm_mfma_supported(const GemmArgs& g) { return g.K % MBK == 0 && g.lda % 4 == 0; }

hipError_t launch_gemm_mfma(const GemmArgs& g, int epi, bool split, hipStream_t s) {
  if (!gemm_mfma_supported(g)) return hipErrorInvalidValue;
  const int bn = epi == EPI_SWIGLU ? MBN / 2 : MBN;
  const int ntiles = (g.N + bn - 1) / bn;
  // 64-row tiles when 128-row tiles would not give every CU a block
  const bool small = ntiles * ((g.M + 127) / 128) < 256;
  const int bm = small ? 64 : 128;
  const dim3 grid(ntiles * ((g.M + bm - 1) / bm)), block(256);
#define SOC_MFMA_CASE(E, SP)                                                     \
  do {                                                                           \
    if (small) hipLaunchKernelGGL((k_gemm_mfma<E, SP, 64>), grid, block, 0, s, g); \
    else hipLaunchKernelGGL((k_gemm_mfma<E, SP, 128>), grid, block, 0, s, g);     \
  } while (0)
  if (split) {
    if (epi == EPI_STORE) SOC_MFMA_CASE(EPI_STORE, true);
    else if (epi == EPI_RESIDUAL) SOC_MFMA_CASE(EPI_RESIDUAL, true);
    else if (epi == EPI_SWIGLU) SOC_MFMA_CASE(EPI_SWIGLU, true);
    else return hipErrorInvalidValue;
  } else {
    if (epi == EPI_STORE) SOC_MFMA_CASE(EPI_STORE, false);
    else if (epi == EPI_RESIDUAL) SOC_MFMA_CASE(EPI_RESIDUAL, false);
    else if (epi == EPI_SWIGLU) SOC_MFMA_CASE(EPI_SWIGLU, false);
    else return hipErrorInvalidValue;
  }
#undef SOC_MFMA_CASE
  return hipGetLastError();
}

}  // namespace soc
