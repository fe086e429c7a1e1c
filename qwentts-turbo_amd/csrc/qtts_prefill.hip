// Backbone prefill on MI355X (gfx950): the S prompt tokens through every layer at once, the
// projections and both attention products on bf16 MFMA with f32 accumulation, K and V written
// straight into the decode kernels' cache layout [layers, 8, max_seq, 128] bf16.
//
// What it replaces: the reference prefills with the qwen_tts PyTorch talker forward in bf16
// (generator.py:209-225: transformers Qwen3DecoderLayer op order, TF/qwen3/modeling_qwen3.py
// :50-64, :140-208, :211-324) and then copies that DynamicCache into the megakernel cache
// (generator.py:245-257, megakernel_backbone.py:285-294); the first group-0 token comes from
// the last position's hidden through the codec head (generator.py:113-117). Every value is
// rounded where that bf16 forward rounds it:
//   xn  = bf16(w * bf16(x * (1 / sqrt(mean(x^2) + eps))))              RMSNorm (:59-64)
//   q,k,v = bf16(W xn); q,k per head through RMSNorm, then
//   rope = bf16(bf16(q * cos) + bf16(rotate_half(q) * sin))            bf16 cos/sin tables
//   s   = scale * (q . k) in f32; att = bf16((sum_j bf16(e^(s_j - m)) v_j) / sum_j e^(s_j - m))
//         with the running max m: the scores and softmax as flash-style attention kernels
//         (torch's sdpa on bf16) keep and round them, normalised after the P V product (eager
//         torch rounds s = bf16(bf16(q . k) * scale) and p = bf16(e / l) before it; :185-208)
//   h1  = bf16(h + bf16(W_o att)); a = bf16(bf16(silu(bf16(W_g xn))) * bf16(W_u xn))
//   h   = bf16(h1 + bf16(W_d a)); hidden = RMSNorm_final(h[S-1]); logits = bf16(W_head hidden)
// The f32 sums run in MFMA order rather than the CPU's, so an f32 result can land on the other
// side of a bf16 rounding boundary now and then; parity is a tolerance, not bit equality.
//
// Kernels (the host loop over layers is in qtts_backbone_prefill below):
//   rmsnorm_kernel   one wave per token
//   gemm_rows_kernel C = A W^T for prompts of at most 128 tokens: all rows in one workgroup, a
//                    32-row weight slice, operands straight into registers (the token operand
//                    in the token-fragment layout its producers write), 4 waves splitting K
//   gemm_dma_kernel  C = A W^T from 256 rows on: 128 x 128 tiles (2 x 2 waves of 64 x 64),
//                    K steps of 64 copied global -> LDS by DMA through 2-3 swizzled stages
//   gemm_kernel      C = A W^T for 129-255 rows and the codec head: 128 x 64 tiles (4 waves,
//                    each 32 rows x 2 MFMA 32x32x16 blocks), K steps of 128, LDS double buffer
//                    + 2 register stages of branch-free loads
//                    All three: split-K over grid.z when the tile grid alone would leave CUs
//                    idle (partials in f32, summed in a fixed order by the reductions);
//                    epilogues: store, residual add, SwiGLU
//   rope_kv_kernel   q/k RMSNorm + interleaved mRoPE, K/V cache write, one workgroup per token
//                    (fused into the split-K reduction of QKV when split: reduce_rope_kernel)
//   reduce_resid_norm_kernel  split-K O / down: sums, residual add and the next RMSNorm per token
//   attn_kernel      causal GQA, 4 waves per (32-query block, query head) splitting the key
//                    blocks: S^T = K Q^T on MFMA (each lane then holds one query's scores, so
//                    the row max and sum stay in the lane and its partner half-wave), one pass
//                    with a running max, O^T += V^T P^T on MFMA with V^T read from the row-major
//                    V block through LDS transpose reads, partials merged in wave order
//   select_kernel    suppress mask + EOS suppression + the decode kernels' wave_select
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include "qwentts_amd.h"
#include "qtts_common.h"
#include "qtts_select.h"

namespace qtts {
namespace pf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float EPS = 1e-6f;                 // Qwen3RMSNorm eps (config rms_norm_eps)
constexpr int BM = 128;                      // GEMM tile rows (columns TN: 64 or 128)
constexpr int GT = 256;                      // GEMM threads (4 waves)
// K step of a TN-column tile: 128 for the 64-column (small-M, latency-bound) tiles, whose short
// K loops then take half the load round trips; 64 for the 128-column tiles
template <int TN> constexpr int bk_of() { return TN == 64 ? 128 : 64; }  // 128-column tiles: gemm_dma_kernel
constexpr int QKVW = 4096;                   // q | k | v row of one token
constexpr int QROW = 136;                    // LDS row of the query block: 128 dims + 16-byte pad
constexpr int MAX_SPLIT = 16;

enum WMode { W_DIRECT, W_QKV, W_O, W_GU, W_DOWN };
enum Epi { E_STORE, E_RESID, E_SWIGLU };

struct GemmArgs {
  const bf16_t* A;                 // [M, K] activations, row stride lda
  int lda;
  const TTSLayerWeights* layers;   // device table (W_QKV .. W_DOWN)
  int layer;
  const bf16_t* B;                 // W_DIRECT: [N, K]
  int M, N, K;                     // N: virtual columns (SwiGLU: gate/up interleaved by 32)
  int kchunk;                      // K range per split (grid.z splits)
  bf16_t* out;
  int ldo;
  const bf16_t* res;               // E_RESID: residual (may alias out)
  int ldr;
  float* part;                     // split-K partials [splits][M][N]
};

// What the QKV GEMM needs to finish a head itself (q/k RMSNorm, RoPE, the K/V cache write);
// kc == nullptr: plain store
struct RopeArgs {
  const bf16_t* cos_t;
  const bf16_t* sin_t;
  const int* pos3;                 // [3][M] (t, h, w) table rows, or nullptr: row = p0 + token
  int p0;
  bf16_t* kc;
  bf16_t* vc;
  int max_seq;
};

__device__ __forceinline__ bf16x8 as_bf8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// bf16 rounding (round to nearest even) with gfx950's conversion instruction
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float rbh(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ bf16_t f2bh(float x) { return __builtin_bit_cast(bf16_t, (__bf16)x); }
__device__ __forceinline__ uint32_t pack_bh(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Token-fragment layout of the row GEMM's token operand (a [rows][K] bf16 matrix of at most RM
// rows, K a multiple of 32, rows allocated in whole 16-row blocks): element (m, k) sits where
// lane (m & 15) + 16 ((k >> 3) & 3) of fragment (m >> 4, k >> 5) holds it in the
// v_mfma_f32_16x16x32_bf16 B operand. A fragment is 64 x 16 contiguous bytes, so the GEMM reads it
// with one fully coalesced load. (Rows of 16 lanes on 16 different rows cost the address unit
// four times the cycles of the same bytes in contiguous order.) Eight consecutive k of one row stay
// together.
__device__ __forceinline__ size_t frag_at(int m, int k, int K) {
  return ((((size_t)(m >> 4) * (K >> 5) + (k >> 5)) * 64 + ((k >> 3) & 3) * 16 + (m & 15)) << 3) + (k & 7);
}

__device__ __forceinline__ const bf16_t* tbl(const TTSLayerWeights* lw, int field) {
  return reinterpret_cast<const bf16_t*>(ld_const(reinterpret_cast<const void* const*>(lw) + field));
}

// x sigmoid(x) in f32 from the hardware exp2 and reciprocal (about 2 ulp of f32 from x / (1 + e^-x),
// far below the bf16 rounding that follows; large |x| gives x or -0 as the exact form does)
__device__ __forceinline__ float silu_f(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

template <int EPI>
__device__ __forceinline__ void epilogue(const GemmArgs& g, int m, int n, float v) {
  if constexpr (EPI == E_STORE) {
    g.out[(size_t)m * g.ldo + n] = f2bh(v);
  } else if constexpr (EPI == E_RESID) {
    const float r = bf2f(g.res[(size_t)m * g.ldr + n]);
    g.out[(size_t)m * g.ldo + n] = f2bh(r + rbh(v));
  }
}

// output column j of the SwiGLU GEMM from its gate and up sums
__device__ __forceinline__ void epilogue_swiglu(const GemmArgs& g, int m, int j, float gs, float us) {
  const float a = rbh(silu_f(rbh(gs)));
  g.out[(size_t)m * g.ldo + j] = f2bh(a * rbh(us));
}

// SwiGLU tiles of TN virtual columns hold TN / 2 outputs: rows [64 q, 64 q + 32) of the tile are
// gate rows and [64 q + 32, 64 q + 64) the up rows of the same 32 outputs, so each wave's two
// 32-column MFMA blocks are a (gate, up) pair in the same lanes. Virtual column n -> weight row:
template <int TN>
__device__ __forceinline__ int swiglu_row(int n, bool& up) {
  const int tt = n / TN, r = n % TN;
  up = ((r >> 5) & 1) != 0;
  return (TN / 2) * tt + 32 * (r >> 6) + (r & 31);
}
// ... and output column j -> its gate virtual column (the up column is 32 further)
template <int TN>
__device__ __forceinline__ int swiglu_gate_col(int j) {
  const int tt = j / (TN / 2), r = j % (TN / 2);
  return TN * tt + 64 * (r >> 5) + (r & 31);
}

// Weight row of virtual column n of a layer projection (SwiGLU: the tile interleave of swiglu_row)
template <int WM, int TN>
__device__ __forceinline__ const bf16_t* weight_row(const GemmArgs& g, const TTSLayerWeights* lw, int n) {
  if constexpr (WM == W_DIRECT) {
    return g.B + (size_t)n * g.K;
  } else if constexpr (WM == W_QKV) {
    return n < 2048 ? tbl(lw, 1) + (size_t)n * g.K
                    : (n < 3072 ? tbl(lw, 2) + (size_t)(n - 2048) * g.K : tbl(lw, 3) + (size_t)(n - 3072) * g.K);
  } else if constexpr (WM == W_O) {
    return tbl(lw, 6) + (size_t)n * g.K;
  } else if constexpr (WM == W_GU) {
    bool up;
    const int row = swiglu_row<TN>(n, up);
    return (up ? tbl(lw, 9) : tbl(lw, 8)) + (size_t)row * g.K;
  } else {
    return tbl(lw, 10) + (size_t)n * g.K;
  }
}

// C = A W^T on a BM x 64 tile (prompts of 129-255 tokens, and the codec head): wave w owns rows
// 32 w .. 32 w + 31 and both 32-column blocks; K steps of 128 through an LDS double buffer fed
// from register stages.
template <int WM, int EPI, int TN>
__global__ void __launch_bounds__(GT, 1) gemm_kernel(const GemmArgs g) {
  static_assert(TN == 64, "the 128-column tiles run in gemm_dma_kernel");
  constexpr int BK = bk_of<TN>();
  constexpr int LROW = BK + 8;                     // LDS row (bf16): 16-byte aligned, skewed banks
  constexpr int CPR = BK / 8;                      // 16-byte chunks per tile row
  constexpr int RPP = GT / CPR;                    // tile rows one pass of the workgroup loads
  constexpr int NAR = BM / RPP;                    // A chunks per thread
  constexpr int NBR = TN / RPP;                    // B chunks per thread
  constexpr int MBW = 1;                           // 32-row blocks per wave
  __shared__ __attribute__((aligned(16))) bf16_t sa[2][BM * LROW];
  __shared__ __attribute__((aligned(16))) bf16_t sb[2][TN * LROW];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * TN;
  const int kbeg = blockIdx.z * g.kchunk, nk = g.kchunk / BK;
  const int lr = t / CPR, lc = (t % CPR) * 8;   // this thread's load row (within RPP) and column
  const int wr0 = 32 * w, wc0 = 0;                // wave's first tile row and column

  // weight rows this thread stages (virtual columns n0 + lr + 32 i)
  const bf16_t* brow[NBR];
  {
    const TTSLayerWeights* lw = g.layers + g.layer;
#pragma unroll
    for (int i = 0; i < NBR; ++i) brow[i] = weight_row<WM, TN>(g, lw, n0 + lr + RPP * i) + kbeg + lc;
  }
  const bf16_t* arow[NAR];
  bool aok[NAR];
#pragma unroll
  for (int i = 0; i < NAR; ++i) {
    const int m = m0 + lr + RPP * i;
    aok[i] = m < g.M;
    arow[i] = g.A + (size_t)(aok[i] ? m : 0) * g.lda + kbeg + lc;
  }

  // NST register stages ahead of the MFMAs (tile kt + NST loads while tile kt computes and tile
  // kt + 1 moves to LDS). Every load is issued unconditionally (rows past M read row 0 and are
  // zeroed afterwards; K steps past the end reload the last one): a load under a branch makes the
  // compiler wait for all outstanding loads instead of just the old ones.
  constexpr int NST = 2;   // a third stage measured 5-10% slower
  u32x4 ra[NST][NAR], rb[NST][NBR];
  auto gload = [&](int k0, u32x4 (&a)[NAR], u32x4 (&b)[NBR]) {
#pragma unroll
    for (int i = 0; i < NAR; ++i) {
      const u32x4 v = ldw(arow[i] + k0);
      a[i] = aok[i] ? v : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < NBR; ++i) b[i] = ldw(brow[i] + k0);
  };
  auto sstore = [&](int buf, const u32x4 (&a)[NAR], const u32x4 (&b)[NBR]) {
#pragma unroll
    for (int i = 0; i < NAR; ++i) *reinterpret_cast<u32x4*>(&sa[buf][(lr + RPP * i) * LROW + lc]) = a[i];
#pragma unroll
    for (int i = 0; i < NBR; ++i) *reinterpret_cast<u32x4*>(&sb[buf][(lr + RPP * i) * LROW + lc]) = b[i];
  };

  f32x16 acc[MBW][2];
#pragma unroll
  for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  const int arow_l = (wr0 + (lane & 31)) * LROW, brow_l = (wc0 + (lane & 31)) * LROW, kh = 8 * (lane >> 5);
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int ko = 16 * kk + kh;
      bf16x8 av[MBW], bv[2];
#pragma unroll
      for (int mb = 0; mb < MBW; ++mb)
        av[mb] = as_bf8(*reinterpret_cast<const u32x4*>(&sa[buf][arow_l + 32 * mb * LROW + ko]));
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        bv[nb] = as_bf8(*reinterpret_cast<const u32x4*>(&sb[buf][brow_l + 32 * nb * LROW + ko]));
#pragma unroll
      for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[mb], bv[nb], acc[mb][nb], 0, 0, 0);
    }
  };
  // one step: tile kt in LDS buffer kt & 1, tile kt + 1 in register stage (kt + 1) % NST, stage
  // kt % NST free (its tile went to LDS in the previous step)
  auto step = [&](int kt, u32x4 (&a0)[NAR], u32x4 (&b0)[NBR], const u32x4 (&a1)[NAR], const u32x4 (&b1)[NBR]) {
    gload(min(kt + NST, nk - 1) * BK, a0, b0);
    compute(kt & 1);
    if (kt + 1 < nk) sstore((kt + 1) & 1, a1, b1);
    __syncthreads();
  };

#pragma unroll
  for (int st = 0; st < NST; ++st) gload(min(st, nk - 1) * BK, ra[st], rb[st]);
  sstore(0, ra[0], rb[0]);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += NST) {
    step(kt, ra[0], rb[0], ra[1], rb[1]);
    if (kt + 1 < nk) step(kt + 1, ra[1], rb[1], ra[0], rb[0]);
  }

  // D layout of a 32x32 block: lane column lane & 31; register r holds row
  // 8 (r >> 2) + 4 (lane >> 5) + (r & 3)
  const int col = lane & 31, hrow = 4 * (lane >> 5);
  if (gridDim.z > 1) {
    float* P = g.part + (size_t)blockIdx.z * g.M * g.N;
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wr0 + 32 * mb + 8 * (r >> 2) + hrow + (r & 3);
          if (m < g.M) P[(size_t)m * g.N + n0 + wc0 + 32 * nb + col] = acc[mb][nb][r];
        }
    return;
  }
#pragma unroll
  for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wr0 + 32 * mb + 8 * (r >> 2) + hrow + (r & 3);
      if (m >= g.M) continue;
      if constexpr (EPI == E_SWIGLU) {
        epilogue_swiglu(g, m, n0 / 2 + wc0 / 2 + col, acc[mb][0][r], acc[mb][1][r]);
      } else {
        epilogue<EPI>(g, m, n0 + wc0 + col, acc[mb][0][r]);
        epilogue<EPI>(g, m, n0 + wc0 + 32 + col, acc[mb][1][r]);
      }
    }
}

// Token-row GEMM for prompts of at most RM tokens: all M rows in one workgroup, a tile of TN
// weight rows (virtual columns). At this size the weights are the only large operand (the token
// rows are at most 256 KB and stay in L2), so the kernel is a weight stream. Each workgroup
// streams its own slice of the weights, and all the operands go straight into registers in the
// v_mfma_f32_16x16x32_bf16 layout, with no LDS staging and no barrier in the K loop:
// - weight block nb is the A operand: lane l holds 8 bf16 of weight row 16 nb + (l & 15) at
//   k = 32 s + 8 (l >> 4);
// - token block mb is the B operand: the same for token row 16 mb + (l & 15), read from the
//   token-fragment layout (frag_at) as one contiguous 1 KB fragment. Blocks past the last row
//   block read the last one, and the sums of rows past M are never stored.
// The 4 waves split the workgroup's K range (g.kchunk = 4 x 32 x NST) into quarters. Each wave
// keeps D steps of loads in flight. The quarter sums meet in LDS and are added in wave order,
// then go through the GEMM's epilogue, or to the split-K partials when grid.z > 1. A SwiGLU
// tile's first TN / 2 weight rows are gate rows of outputs TN / 2 x tile + 0 .. TN / 2 - 1, its
// last TN / 2 the up rows of the same outputs; its output (the down projection's input) is
// written in the token-fragment layout. This kernel never splits SwiGLU.
constexpr int RM = 128;

template <int WM, int EPI, int TN, int NST>
__global__ void __launch_bounds__(GT, 2) gemm_rows_kernel(const GemmArgs g) {
  static_assert(WM != W_DIRECT && TN % 32 == 0, "row GEMM: layer weights, 16-row blocks in pairs");
  constexpr int NB = TN / 16, MB = RM / 16;
  constexpr int D = NST < 4 ? NST : 4;
  constexpr int RROW = TN + 4;                 // f32 LDS row of a quarter sum (16-byte aligned)
  __shared__ __attribute__((aligned(16))) float red[4][RM * RROW];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, i = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * TN;
  const int k0 = blockIdx.z * g.kchunk + w * (32 * NST) + 8 * kg;
  const TTSLayerWeights* lw = g.layers + g.layer;
  const bf16_t* wp[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = n0 + 16 * nb + i;
    const bf16_t* p;
    if constexpr (WM == W_QKV) {
      p = n < 2048 ? tbl(lw, 1) + (size_t)n * g.K
                   : (n < 3072 ? tbl(lw, 2) + (size_t)(n - 2048) * g.K : tbl(lw, 3) + (size_t)(n - 3072) * g.K);
    } else if constexpr (WM == W_O) {
      p = tbl(lw, 6) + (size_t)n * g.K;
    } else if constexpr (WM == W_GU) {
      const int j = n0 / 2 + 16 * (nb % (NB / 2)) + i;
      p = (nb < NB / 2 ? tbl(lw, 8) : tbl(lw, 9)) + (size_t)j * g.K;
    } else {
      p = tbl(lw, 10) + (size_t)n * g.K;
    }
    wp[nb] = p + k0;
  }
  const bf16_t* xp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    xp[mb] = g.A + (((size_t)min(mb, (g.M - 1) >> 4) * (g.K >> 5) + ((k0 - 8 * kg) >> 5)) * 64 + lane) * 8;

  u32x4 wr[D][NB], xr[D][MB];
  f32x4 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < D; ++s) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) wr[s][nb] = ldw(wp[nb] + 32 * s);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[s][mb] = ldw(xp[mb] + 512 * s);
  }
#pragma unroll
  for (int s = 0; s < NST; ++s) {
    const int d = s % D;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(wr[d][nb]), as_bf8(xr[d][mb]), acc[nb][mb], 0, 0, 0);
    if (s + D < NST) {   // compile-time after unrolling
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) wr[d][nb] = ldw(wp[nb] + 32 * (s + D));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) xr[d][mb] = ldw(xp[mb] + 512 * (s + D));
    }
  }

  // D layout: lane l holds weight rows 4 (l >> 4) + e of token column l & 15
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      *reinterpret_cast<f32x4*>(&red[w][(16 * mb + i) * RROW + 16 * nb + 4 * kg]) = acc[nb][mb];
  __syncthreads();
  auto qsum = [&](int off) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(&red[0][off]);
    const f32x4 b = *reinterpret_cast<const f32x4*>(&red[1][off]);
    const f32x4 c = *reinterpret_cast<const f32x4*>(&red[2][off]);
    const f32x4 e = *reinterpret_cast<const f32x4*>(&red[3][off]);
    return ((a + b) + c) + e;
  };
  if constexpr (EPI == E_SWIGLU) {
    constexpr int C4 = TN / 8;                 // groups of 4 outputs per token row
#pragma unroll
    for (int q = t; q < RM * C4; q += GT) {
      const int m = q / C4, c = 4 * (q % C4);
      if (m >= g.M) break;
      const f32x4 gs = qsum(m * RROW + c), us = qsum(m * RROW + TN / 2 + c);
      u32x2 o;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float a0 = rbh(silu_f(rbh(gs[2 * e]))) * rbh(us[2 * e]);
        const float a1 = rbh(silu_f(rbh(gs[2 * e + 1]))) * rbh(us[2 * e + 1]);
        o[e] = pack_bh(a0, a1);
      }
      *reinterpret_cast<u32x2*>(g.out + frag_at(m, n0 / 2 + c, g.ldo)) = o;
    }
  } else {
    constexpr int C4 = TN / 4;
#pragma unroll
    for (int q = t; q < RM * C4; q += GT) {
      const int m = q / C4, c = 4 * (q % C4);
      if (m >= g.M) break;
      const f32x4 v = qsum(m * RROW + c);
      if (gridDim.z > 1) {
        *reinterpret_cast<f32x4*>(g.part + (size_t)blockIdx.z * g.M * g.N + (size_t)m * g.N + n0 + c) = v;
      } else if constexpr (EPI == E_RESID) {
        const u32x2 r = *reinterpret_cast<const u32x2*>(g.res + (size_t)m * g.ldr + n0 + c);
        u32x2 o;
        o[0] = pack_bh(bflo(r[0]) + rbh(v[0]), bfhi(r[0]) + rbh(v[1]));
        o[1] = pack_bh(bflo(r[1]) + rbh(v[2]), bfhi(r[1]) + rbh(v[3]));
        *reinterpret_cast<u32x2*>(g.out + (size_t)m * g.ldo + n0 + c) = o;
      } else {
        u32x2 o;
        o[0] = pack_bh(v[0], v[1]);
        o[1] = pack_bh(v[2], v[3]);
        *reinterpret_cast<u32x2*>(g.out + (size_t)m * g.ldo + n0 + c) = o;
      }
    }
  }
}

#define QTTS_PF_INLINE __attribute__((always_inline))
typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// C = A W^T on a 128 x 128 tile (prompts from 256 tokens on), K steps of 64, with the operands
// copied from global memory straight into LDS (global_load_lds_dwordx4: each wave instruction
// writes 64 x 16 bytes at a wave-uniform LDS address) through NS stages. No register staging and
// no LDS store instructions; one barrier per K step.
// - LDS tile layout: row r of a stage holds its 8 16-byte k-chunks with chunk c at position
//   c ^ (r & 7). A DMA instruction covers 8 rows; lane l writes position l & 7 of row l >> 3 and
//   so loads chunk (l & 7) ^ (r & 7) of that row: 8 lanes read one 128-byte row segment.
// - The XOR swizzle makes the MFMA operand reads (32 rows at one chunk) conflict-free.
// - Waves form 2 x 2; wave w owns rows 64 (w & 1) .. + 63 and columns 64 (w >> 1) .. + 63 (two
//   32 x 32 MFMA blocks each way), as in gemm_kernel's 128-column tile, and the epilogues match.
// - Rows past M read row M - 1; their sums are never stored.
// - The wait before each barrier counts this wave's DMA instructions still in flight: the
//   compiler does not track LDS writes made by DMA.
// - Unsplit QKV with rope arguments: a tile is one head of 128 tokens, and the epilogue finishes
//   it as rope_kv_apply does: bf16 tile through LDS, then two threads per token (32 channel pairs
//   (d, d + 64) each) for the q/k RMSNorm and the interleaved mRoPE. q goes back to the QKV rows;
//   k and v go to the cache.
template <int WM, int EPI, int NS>
__global__ void __launch_bounds__(GT, NS <= 2 ? 2 : 1) gemm_dma_kernel(const GemmArgs g, const RopeArgs ra) {
  constexpr int TN = 128, TM = 128, BK = 64;
  constexpr int STAGE = (TM + TN) * BK * 2;        // bytes of one stage (A then B)
  constexpr int NIA = TM * BK * 2 / 1024 / 4;      // DMA instructions per wave for A (4)
  constexpr int NIB = TN * BK * 2 / 1024 / 4;      // ... and for B (4)
  constexpr int NIW = NIA + NIB;
  static_assert(NS >= 2 && NS <= 4 && NIW <= 15, "stages / vmcnt field");
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
  const int kbeg = blockIdx.z * g.kchunk, nk = g.kchunk / BK;
  const TTSLayerWeights* lw = g.layers + g.layer;

  // this lane's source rows: instruction i of the wave covers tile rows 8 (NIA w + i) .. + 7
  const bf16_t* asrc[NIA];
  const bf16_t* bsrc[NIB];
#pragma unroll
  for (int i = 0; i < NIA; ++i) {
    const int r = 8 * (NIA * w + i) + (lane >> 3);
    const int c = (lane & 7) ^ (r & 7);
    asrc[i] = g.A + (size_t)min(m0 + r, g.M - 1) * g.lda + kbeg + 8 * c;
  }
#pragma unroll
  for (int i = 0; i < NIB; ++i) {
    const int r = 8 * (NIB * w + i) + (lane >> 3);
    const int c = (lane & 7) ^ (r & 7);
    bsrc[i] = weight_row<WM, TN>(g, lw, n0 + r) + kbeg + 8 * c;
  }
  // stage s <- K step kt (clamped: steps past the end reload the last one)
  auto issue = [&](int s, int kt) QTTS_PF_INLINE {
    const int k = BK * min(kt, nk - 1);
    char* base = lds + s * STAGE;
#pragma unroll
    for (int i = 0; i < NIA; ++i)
      __builtin_amdgcn_global_load_lds((gvoid_t*)(asrc[i] + k), (lvoid_t*)(base + 1024 * (NIA * w + i)), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < NIB; ++i)
      __builtin_amdgcn_global_load_lds((gvoid_t*)(bsrc[i] + k), (lvoid_t*)(base + TM * BK * 2 + 1024 * (NIB * w + i)),
                                       16, 0, 0);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;
  const int wr0 = 64 * (w & 1), wc0 = 64 * (w >> 1), hk = lane >> 5;
  // byte offset of (row r, chunk c) in a stage's A or B part
  auto at = [](int r, int c) { return (r * 8 + (c ^ (r & 7))) * 16; };
  auto compute = [&](int s) QTTS_PF_INLINE {
    const char* a = lds + s * STAGE;
    const char* b = a + TM * BK * 2;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c = 2 * kk + hk;
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) av[mb] = as_bf8(*reinterpret_cast<const u32x4*>(a + at(wr0 + 32 * mb + (lane & 31), c)));
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) bv[nb] = as_bf8(*reinterpret_cast<const u32x4*>(b + at(wc0 + 32 * nb + (lane & 31), c)));
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[mb], bv[nb], acc[mb][nb], 0, 0, 0);
    }
  };

#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue(s, s);
  for (int kt = 0; kt < nk; ++kt) {
    // this wave's DMA for step kt has landed when at most (NS - 2) stages' instructions remain
    __builtin_amdgcn_s_waitcnt(0x0F70 | ((NS - 2) * NIW));
    __builtin_amdgcn_s_barrier();   // every wave's step kt is in LDS; step kt - 1's buffer is free
    issue((kt + NS - 1) % NS, kt + NS - 1);
    compute(kt % NS);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);   // no DMA may still target LDS when the workgroup ends

  const int col = lane & 31, hrow = 4 * (lane >> 5);
  if constexpr (WM == W_QKV && EPI == E_STORE) {
    if (ra.kc != nullptr) {
      constexpr int TR = HDIM + 8;   // bf16 row of the staged head tile (16-byte aligned, skewed)
      bf16_t* T = reinterpret_cast<bf16_t*>(lds);
      __syncthreads();   // every wave's DMA has landed and its last MFMA reads are done
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            T[(wr0 + 32 * mb + 8 * (r >> 2) + hrow + (r & 3)) * TR + wc0 + 32 * nb + col] = f2bh(acc[mb][nb][r]);
      __syncthreads();
      const int head = n0 / HDIM;   // q heads 0..15, k heads 16..23, v heads 24..31
      if (head >= NQH + NKVH) {
        bf16_t* vbase = ra.vc + ((size_t)g.layer * NKVH + (head - NQH - NKVH)) * ra.max_seq * HDIM;
        for (int q = t; q < TM * 16; q += GT) {
          const int row = q >> 4, ch = 8 * (q & 15), m = m0 + row;
          if (m < g.M)
            *reinterpret_cast<u32x4*>(vbase + (size_t)(ra.p0 + m) * HDIM + ch) =
                *reinterpret_cast<const u32x4*>(&T[row * TR + ch]);
        }
        return;
      }
      const int row = t >> 1, hf = t & 1, m = min(m0 + row, g.M - 1);
      const bf16_t* tr = &T[row * TR + 32 * hf];
      float ss = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(tr + 8 * c);
        const u32x4 b = *reinterpret_cast<const u32x4*>(tr + 64 + 8 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ss += bflo(a[e]) * bflo(a[e]) + bflo(b[e]) * bflo(b[e]);
          ss += bfhi(a[e]) * bfhi(a[e]) + bfhi(b[e]) * bfhi(b[e]);
        }
      }
      ss += __shfl_xor(ss, 1, 64);
      const float rs = 1.0f / sqrtf(ss / (float)HDIM + EPS);
      const bool isq = head < NQH;
      const bf16_t* gn = tbl(lw, isq ? 4 : 5);
      // table rows of the three sections (t, h, w); channel d < 60 takes h when d % 3 == 1 and w
      // when d % 3 == 2, every other channel t (the same row for d and d + 64)
      const int pos = ra.p0 + m;
      int rsec[3];
#pragma unroll
      for (int j = 0; j < 3; ++j) rsec[j] = ra.pos3 ? min(max(ra.pos3[j * g.M + m], 0), ra.max_seq - 1) : pos;
      bf16_t* dst = isq ? g.out + (size_t)m * g.ldo + n0
                        : ra.kc + (((size_t)g.layer * NKVH + (head - NQH)) * ra.max_seq + pos) * HDIM;
      // 8 channel pairs (d0 + e, d0 + 64 + e); cs/sn: this chunk's cos and sin for d and d + 64,
      // already picked per section
      auto finish = [&](int c, const float (&c0)[8], const float (&c1)[8], const float (&s0)[8],
                        const float (&s1)[8], const u32x4& g0, const u32x4& g1) QTTS_PF_INLINE {
        const int d0 = 32 * hf + 8 * c;
        const u32x4 a = *reinterpret_cast<const u32x4*>(tr + 8 * c);
        const u32x4 b = *reinterpret_cast<const u32x4*>(tr + 64 + 8 * c);
        u32x4 o0, o1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float r0[2], r1[2];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int k = 2 * e + h2;
            const float x0 = h2 ? bfhi(a[e]) : bflo(a[e]), x1 = h2 ? bfhi(b[e]) : bflo(b[e]);
            const float ga = h2 ? bfhi(g0[e]) : bflo(g0[e]), gb = h2 ? bfhi(g1[e]) : bflo(g1[e]);
            const float y0 = rbh(ga * rbh(x0 * rs)), y1 = rbh(gb * rbh(x1 * rs));
            r0[h2] = rbh(y0 * c0[k]) + rbh(-y1 * s0[k]);
            r1[h2] = rbh(y1 * c1[k]) + rbh(y0 * s1[k]);
          }
          o0[e] = pack_bh(r0[0], r0[1]);
          o1[e] = pack_bh(r1[0], r1[1]);
        }
        if (m0 + row < g.M) {
          *reinterpret_cast<u32x4*>(dst + d0) = o0;
          *reinterpret_cast<u32x4*>(dst + d0 + 64) = o1;
        }
      };
      auto unpack8 = [](const u32x4& v, float (&f)[8]) QTTS_PF_INLINE {
#pragma unroll
        for (int e = 0; e < 4; ++e) { f[2 * e] = bflo(v[e]); f[2 * e + 1] = bfhi(v[e]); }
      };
      if (ra.pos3 == nullptr) {
        // one table row per token: every load of the 4 chunks issued before the first use
        const bf16_t* cr = ra.cos_t + (size_t)pos * HDIM + 32 * hf;
        const bf16_t* sr = ra.sin_t + (size_t)pos * HDIM + 32 * hf;
        u32x4 vc0[4], vc1[4], vs0[4], vs1[4], vg0[4], vg1[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          vc0[c] = ldw(cr + 8 * c); vc1[c] = ldw(cr + 64 + 8 * c);
          vs0[c] = ldw(sr + 8 * c); vs1[c] = ldw(sr + 64 + 8 * c);
          vg0[c] = ldw(gn + 32 * hf + 8 * c); vg1[c] = ldw(gn + 64 + 32 * hf + 8 * c);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float c0[8], c1[8], s0[8], s1[8];
          unpack8(vc0[c], c0); unpack8(vc1[c], c1); unpack8(vs0[c], s0); unpack8(vs1[c], s1);
          finish(c, c0, c1, s0, s1, vg0[c], vg1[c]);
        }
      } else {
#pragma unroll 1
        for (int c = 0; c < 4; ++c) {
          const int d0 = 32 * hf + 8 * c;
          u32x4 cs0[3], cs1[3], sn0[3], sn1[3];
#pragma unroll
          for (int j = 0; j < 3; ++j) {
            const size_t ro = (size_t)rsec[j] * HDIM + d0;
            cs0[j] = ldw(ra.cos_t + ro); cs1[j] = ldw(ra.cos_t + ro + 64);
            sn0[j] = ldw(ra.sin_t + ro); sn1[j] = ldw(ra.sin_t + ro + 64);
          }
          float c0[8], c1[8], s0[8], s1[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int d = d0 + k, sec = (d < 60 && d % 3 == 1) ? 1 : ((d < 60 && d % 3 == 2) ? 2 : 0);
            auto pick = [&](const u32x4 (&v)[3]) {
              const uint32_t wv = sec == 0 ? v[0][k >> 1] : (sec == 1 ? v[1][k >> 1] : v[2][k >> 1]);
              return (k & 1) ? bfhi(wv) : bflo(wv);
            };
            c0[k] = pick(cs0); c1[k] = pick(cs1); s0[k] = pick(sn0); s1[k] = pick(sn1);
          }
          finish(c, c0, c1, s0, s1, ldw(gn + d0), ldw(gn + d0 + 64));
        }
      }
      return;
    }
  }
  if (gridDim.z > 1) {
    float* P = g.part + (size_t)blockIdx.z * g.M * g.N;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wr0 + 32 * mb + 8 * (r >> 2) + hrow + (r & 3);
          if (m < g.M) P[(size_t)m * g.N + n0 + wc0 + 32 * nb + col] = acc[mb][nb][r];
        }
    return;
  }
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wr0 + 32 * mb + 8 * (r >> 2) + hrow + (r & 3);
      if (m >= g.M) continue;
      if constexpr (EPI == E_SWIGLU) {
        epilogue_swiglu(g, m, n0 / 2 + wc0 / 2 + col, acc[mb][0][r], acc[mb][1][r]);
      } else {
        epilogue<EPI>(g, m, n0 + wc0 + col, acc[mb][0][r]);
        epilogue<EPI>(g, m, n0 + wc0 + 32 + col, acc[mb][1][r]);
      }
    }
}

// Sums in split order of the partials at p + z stride, z < splits: 4 NQ consecutive floats
// (NQ 16-byte loads per split). The loads go out in groups of G splits before any of them is
// added (each clamped to the last split, so an unconditional load from a valid address): the
// group's round trips overlap, where a rolled loop waits for each load before it issues the next.
// The additions run in split order, so the sums are the ones of a plain loop, bit for bit.
template <int G, int NQ>
__device__ __forceinline__ void sum_splits(const float* p, size_t stride, int splits, float (&s)[4 * NQ]) {
#pragma unroll
  for (int i = 0; i < 4 * NQ; ++i) s[i] = 0.0f;
  for (int z0 = 0; z0 < splits; z0 += G) {
    u32x4 v[G][NQ];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        v[j][q] = *reinterpret_cast<const u32x4*>(p + (size_t)min(z0 + j, splits - 1) * stride + 4 * q);
    // every load of the group is issued here: the compiler may not sink one into a later branch
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int q = 0; q < NQ; ++q) asm volatile("" : "+v"(v[j][q]));
    // a clamped duplicate adds -0.0, the exact identity of IEEE addition, so the sum is the one of
    // the valid splits alone
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const bool ok = z0 + j < splits;
#pragma unroll
      for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * q + e] += ok ? __uint_as_float(v[j][q][e]) : -0.0f;
    }
  }
}

// Sum of the split-K partials in split order, then the GEMM's epilogue; four consecutive
// outputs per thread (16-byte partial loads; a SwiGLU group of four lies in one 32-column block).
template <int EPI, int TN>
__global__ void __launch_bounds__(256) reduce_kernel(const GemmArgs g, int splits) {
  const int nout = EPI == E_SWIGLU ? g.N / 2 : g.N;
  const long idx = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (idx >= (long)g.M * nout) return;
  const int m = (int)(idx / nout), j = (int)(idx % nout);
  const size_t stride = (size_t)g.M * g.N;
  const float* P = g.part + (size_t)m * g.N;
  if constexpr (EPI == E_SWIGLU) {
    const int nv = swiglu_gate_col<TN>(j);
    float gs[4], us[4];
    sum_splits<4, 1>(P + nv, stride, splits, gs);
    sum_splits<4, 1>(P + nv + 32, stride, splits, us);
#pragma unroll
    for (int e = 0; e < 4; ++e) epilogue_swiglu(g, m, j + e, gs[e], us[e]);
  } else {
    float v[4];
    sum_splits<4, 1>(P + j, stride, splits, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) epilogue<EPI>(g, m, j + e, v[e]);
  }
}

// RMSNorm of M token rows (row stride ldx) into bf16 rows (stride ldo), one wave per token;
// the gain comes from field `field` of layer `layer` of the device table, or `gain` when the
// table is null. out_f32 (optional) receives the bf16 result widened to f32.
__global__ void __launch_bounds__(256) rmsnorm_kernel(const bf16_t* x, int ldx, const TTSLayerWeights* layers,
                                                      int layer, int field, const bf16_t* gain, bf16_t* out,
                                                      int ldo, float* out_f32, int M, int frag) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const bf16_t* w = layers ? tbl(layers + layer, field) : gain;
  const bf16_t* xr = x + (size_t)m * ldx;
  u32x4 v[2];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    v[k] = ldw(xr + 8 * (lane + 64 * k));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = bflo(v[k][e]), b = bfhi(v[k][e]);
      ss += a * a + b * b;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float rs = 1.0f / sqrtf(ss / (float)HID + EPS);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e0 = 8 * (lane + 64 * k);
    const u32x4 gw = ldw(w + e0);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = rbf(bflo(gw[e]) * rbf(bflo(v[k][e]) * rs));
      const float b = rbf(bfhi(gw[e]) * rbf(bfhi(v[k][e]) * rs));
      o[e] = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
      if (out_f32) {
        out_f32[e0 + 2 * e] = a;
        out_f32[e0 + 2 * e + 1] = b;
      }
    }
    if (out) *reinterpret_cast<u32x4*>(out + (frag ? frag_at(m, e0, ldo) : (size_t)m * ldo + e0)) = o;
  }
}

// Per token: q/k head RMSNorm (field 4 / 5 gains), interleaved mRoPE from the bf16 tables, the
// rotated q written to qdst, the rotated k and the v of every KV head written to the cache at
// position p0 + s. Lane j of a wave handles channels j and j + 64 (the rotate_half pair). Run by
// a whole 256-thread workgroup on token s's q | k | v row `src` (global memory or LDS). The table
// and gain values come first (rope_inputs), so a caller can issue those loads before it builds
// the row.
struct RopeIn { float c0, c1, s0, s1, gq0, gq1, gk0, gk1; };

__device__ __forceinline__ RopeIn rope_inputs(int s, const TTSLayerWeights* layers, int layer, const bf16_t* cos_t,
                                              const bf16_t* sin_t, const int* pos3, int p0, int S, int max_seq) {
  const int lane = threadIdx.x & 63;
  const int sec = (lane < 60 && lane % 3 == 1) ? 1 : ((lane < 60 && lane % 3 == 2) ? 2 : 0);
  // table row of this channel's section (clamped into the table: a caller's out-of-range
  // position must not read outside it)
  const int row = pos3 ? min(max(pos3[sec * S + s], 0), max_seq - 1) : p0 + s;
  const TTSLayerWeights* lw = layers + layer;
  const bf16_t* qn = tbl(lw, 4);
  const bf16_t* kn = tbl(lw, 5);
  RopeIn r;
  r.c0 = ldbf(cos_t + (size_t)row * HDIM + lane);
  r.c1 = ldbf(cos_t + (size_t)row * HDIM + lane + 64);
  r.s0 = ldbf(sin_t + (size_t)row * HDIM + lane);
  r.s1 = ldbf(sin_t + (size_t)row * HDIM + lane + 64);
  r.gq0 = ldbf(qn + lane); r.gq1 = ldbf(qn + lane + 64);
  r.gk0 = ldbf(kn + lane); r.gk1 = ldbf(kn + lane + 64);
  return r;
}

__device__ __forceinline__ void rope_kv_apply(const RopeIn& r, const bf16_t* src, bf16_t* qdst, int s, int layer,
                                              int p0, bf16_t* kc, bf16_t* vc, int max_seq) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int pos = p0 + s;
  // wave w takes heads w + 4 k (k < 6): q heads for k < 4, k heads 16 + w, 20 + w for k = 4, 5;
  // every load is issued before the first reduction, the six reductions interleave
  constexpr int HPW = (NQH + NKVH) / 4;
  float x0[HPW], x1[HPW], ss[HPW];
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const bf16_t* hp = src + (w + 4 * k) * HDIM;
    x0[k] = bf2f(hp[lane]);
    x1[k] = bf2f(hp[lane + 64]);
  }
#pragma unroll
  for (int k = 0; k < HPW; ++k) ss[k] = x0[k] * x0[k] + x1[k] * x1[k];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
    for (int k = 0; k < HPW; ++k) ss[k] += __shfl_xor(ss[k], o, 64);
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const float rs = 1.0f / sqrtf(ss[k] / (float)HDIM + EPS);
    const float y0 = rbh((k < 4 ? r.gq0 : r.gk0) * rbh(x0[k] * rs));
    const float y1 = rbh((k < 4 ? r.gq1 : r.gk1) * rbh(x1[k] * rs));
    const bf16_t o0 = f2bh(rbh(y0 * r.c0) + rbh(-y1 * r.s0));
    const bf16_t o1 = f2bh(rbh(y1 * r.c1) + rbh(y0 * r.s1));
    bf16_t* dst = k < 4 ? qdst + (w + 4 * k) * HDIM
                        : kc + (((size_t)layer * NKVH + (w + 4 * (k - 4))) * max_seq + pos) * HDIM;
    dst[lane] = o0;
    dst[lane + 64] = o1;
  }
  // v: 8 heads x 128 = 1024 values, 4 per thread
  const int i0 = 4 * threadIdx.x;
  const int kvh = i0 >> 7, d = i0 & 127;
  const u32x2 vv = *reinterpret_cast<const u32x2*>(src + 3072 + i0);
  *reinterpret_cast<u32x2*>(vc + (((size_t)layer * NKVH + kvh) * max_seq + pos) * HDIM + d) = vv;
}

__global__ void __launch_bounds__(256) rope_kv_kernel(bf16_t* qkv, const TTSLayerWeights* layers, int layer,
                                                      const bf16_t* cos_t, const bf16_t* sin_t, const int* pos3,
                                                      int p0, int S, bf16_t* kc, bf16_t* vc, int max_seq) {
  const RopeIn r = rope_inputs(blockIdx.x, layers, layer, cos_t, sin_t, pos3, p0, S, max_seq);
  bf16_t* row = qkv + (size_t)blockIdx.x * QKVW;
  rope_kv_apply(r, row, row, blockIdx.x, layer, p0, kc, vc, max_seq);   // q rotated in place
}

// Split-K QKV: token m's 4096 sums in split order -> bf16 q | k | v row in LDS, then the q/k-norm,
// RoPE and cache write on it, the rotated q to the token's QKV row (one launch instead of a
// reduction and a rope pass). The table and gain loads go out before the partial sums.
__global__ void __launch_bounds__(256) reduce_rope_kernel(const GemmArgs g, int splits, const bf16_t* cos_t,
                                                          const bf16_t* sin_t, const int* pos3, int p0, bf16_t* kc,
                                                          bf16_t* vc, int max_seq) {
  __shared__ __attribute__((aligned(16))) bf16_t srow[QKVW];
  const int m = blockIdx.x;
  const size_t stride = (size_t)g.M * g.N;
  const float* P = g.part + (size_t)m * g.N;
  const RopeIn r = rope_inputs(m, g.layers, g.layer, cos_t, sin_t, pos3, p0, g.M, max_seq);
  // thread t: elements 16 t .. 16 t + 15, in 16-byte loads
  const int n0 = 16 * threadIdx.x;
  float v[16];
  sum_splits<2, 4>(P + n0, stride, splits, v);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bh(v[8 * q + 2 * e], v[8 * q + 2 * e + 1]);
    *reinterpret_cast<u32x4*>(srow + n0 + 8 * q) = o;
  }
  __syncthreads();   // the row is read back by other threads of the workgroup
  rope_kv_apply(r, srow, g.out + (size_t)m * g.ldo, m, g.layer, p0, kc, vc, max_seq);
}

// Split-K O or down projection of token m: sums in split order, residual add in place
// (h = bf16(h + bf16(sum))), then the RMSNorm of the new row with gain field `field` of layer
// `nlayer` into xn (skipped when nlayer < 0): one launch instead of a reduction and a norm.
__global__ void __launch_bounds__(256) reduce_resid_norm_kernel(const GemmArgs g, int splits, int nlayer, int field,
                                                                bf16_t* xn, int frag) {
  __shared__ float red[4];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const size_t stride = (size_t)g.M * g.N;
  const float* P = g.part + (size_t)m * g.N + 4 * t;
  bf16_t* hr = g.out + (size_t)m * g.ldo + 4 * t;
  const u32x2 rv = *reinterpret_cast<const u32x2*>(g.res + (size_t)m * g.ldr + 4 * t);
  float hv[4];
  {
    float sv[4];
    sum_splits<8, 1>(P, stride, splits, sv);
    hv[0] = rbh(bflo(rv[0]) + rbh(sv[0]));
    hv[1] = rbh(bfhi(rv[0]) + rbh(sv[1]));
    hv[2] = rbh(bflo(rv[1]) + rbh(sv[2]));
    hv[3] = rbh(bfhi(rv[1]) + rbh(sv[3]));
  }
  u32x2 hp;
  hp[0] = pack_bh(hv[0], hv[1]);
  hp[1] = pack_bh(hv[2], hv[3]);
  *reinterpret_cast<u32x2*>(hr) = hp;
  if (nlayer < 0) return;
  float ss = hv[0] * hv[0] + hv[1] * hv[1] + hv[2] * hv[2] + hv[3] * hv[3];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if (lane == 0) red[t >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float rs = 1.0f / sqrtf(ss / (float)HID + EPS);
  const u32x2 gw = *reinterpret_cast<const u32x2*>(tbl(g.layers + nlayer, field) + 4 * t);
  u32x2 o;
  o[0] = pack_bh(bflo(gw[0]) * rbh(hv[0] * rs), bfhi(gw[0]) * rbh(hv[1] * rs));
  o[1] = pack_bh(bflo(gw[1]) * rbh(hv[2] * rs), bfhi(gw[1]) * rbh(hv[3] * rs));
  *reinterpret_cast<u32x2*>(xn + (frag ? frag_at(m, 4 * t, HID) : (size_t)m * HID + 4 * t)) = o;
}

// Causal GQA attention of S queries (positions p0 .. p0 + S - 1) over cache positions
// 0 .. p0 + S - 1, one workgroup of AW waves per (32-query block, query head); wave w takes the
// 32-key blocks kb = w, w + AW, ... in one pass with a running (online) softmax:
//   * S^T = K Q^T on MFMA 32x32x16 (A = the K block staged in the wave's LDS rows, B = Q^T from
//     the block's queries in LDS): lane (half hf, column c) holds query 32 qb + c's scores for
//     keys 8 (r >> 2) + 4 hf + (r & 3), r < 16, so a query's row max and sum stay in the lane and
//     its partner half-wave. The scores stay in f32 and the scale goes into the exponent:
//     e^(s - m) = 2^((q . k - m') scale log2 e) for the unscaled running max m'.
//   * The running max m moves to m' = max(m, block max); O^T and the sum l scale by e^(m - m')
//     (skipped when no query of the wave moved); p = e^(s - m') rounded to bf16 is the B operand
//     of O^T += V^T P^T, reusing the score registers in place (k-index 8 hf + j of step kk2 is key
//     16 kk2 + 8 (j >> 2) + 4 hf + (j & 3)); l sums the f32 e^(s - m').
//   * V^T comes from the V block staged row-major (16-byte writes) through the LDS transpose read
//     ds_read_b64_tr_b16: in each 16-lane group, with M[l][j] = the 4 bf16 at lane l's address,
//     lane i receives M[4 j + (i >> 2)][i & 3], j < 4. Lane i of group g (hf = g >> 1) passes
//     row 16 kk2 + 4 hf (+ 8) + (i >> 2), columns 32 mb + 16 (g & 1) + 4 (i & 3): it receives
//     dims 32 mb + 16 (g & 1) + i, keys 16 kk2 + 4 hf (+ 8) + 0..3, the A operand of O^T.
// The softmax normalisation comes last (att = bf16(O / l)), as in flash-style kernels; the waves'
// (m, l, O^T) merge through LDS in wave order. Grid: 16 x (query blocks) workgroups, KV head =
// linear id mod 8 (one head per XCD's L2), the longest query blocks first.
constexpr int AW = 4;
constexpr int VROW = 160;     // LDS row of a staged V block (bf16): 320 B puts the 4 rows one
                              // transpose read touches 16 banks apart
constexpr int WST = 32 * VROW;                      // a wave's staging region (K block, then V)
constexpr int ATT_Q = 32 * QROW;                    // the query block
constexpr int ATT_SMEM = std::max((ATT_Q + AW * WST) * 2, (AW - 1) * HDIM * 32 * 4 + AW * 2 * 32 * 4);
static_assert(32 * QROW <= WST, "a wave's LDS region holds its staged K block");

typedef short v4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr16(const bf16_t* p) {
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)((__attribute__((address_space(3))) void*)p));
  return __builtin_bit_cast(u32x2, r);
}

__global__ void __launch_bounds__(64 * AW, 2) attn_kernel(const bf16_t* qkv, const bf16_t* kc, const bf16_t* vc,
                                                       int layer, int max_seq, int p0, int S, bf16_t* att,
                                                       float scale, int frag) {
  __shared__ __attribute__((aligned(16))) char smem[ATT_SMEM];
  bf16_t* sq = reinterpret_cast<bf16_t*>(smem);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hf = lane >> 5, c = lane & 31;
  // XCD-aware order: workgroups go to the XCDs round-robin by linear id, so id & 7 picks the KV
  // head and each XCD's L2 holds one head's K and V; within it, the longest query blocks first
  const int nqb = (S + 31) / 32, id = blockIdx.x;
  const int kvh = id & 7, rest = id >> 3;
  const int hq = 2 * kvh + (rest & 1), qb = nqb - 1 - (rest >> 1);
  const int i = 32 * qb + c;
  const bool qok = i < S;
  const int qpos = p0 + i;
  const int last = p0 + min(S, 32 * qb + 32) - 1;   // last key any query of the block sees
  const int nkb = last / 32 + 1;
  bf16_t* st = sq + ATT_Q + w * WST;   // the wave's K block, then its V block

  // the block's 32 query rows (512 16-byte chunks) go to LDS once
#pragma unroll
  for (int j = 0; j < 512 / (64 * AW); ++j) {
    const int ch = threadIdx.x + 64 * AW * j, qrow = ch >> 4, qcol = 8 * (ch & 15);
    const int qi = 32 * qb + qrow;
    const u32x4 v = ldw(qkv + (size_t)(qi < S ? qi : 0) * QKVW + hq * HDIM + qcol);   // clamped row
    *reinterpret_cast<u32x4*>(&sq[qrow * QROW + qcol]) = qi < S ? v : u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  const size_t hbase = ((size_t)layer * NKVH + kvh) * max_seq * HDIM;
  const bf16_t* kb_ = kc + hbase;
  const bf16_t* vb_ = vc + hbase;

  // K and V blocks (32 keys x 128 dims each) in 8 coalesced 1 KB rounds, issued a block ahead:
  // round r, lane j loads key 32 kb + 4 r + (j >> 4), dims 8 (j & 15) .. + 7. Loads are
  // unconditional from a clamped row (row 0 past `last`) and staged as loaded: a load or a store
  // under a branch makes the compiler wait for every outstanding load, the prefetch included. Keys
  // past `last` are past every query of the block, so their scores are masked to -inf and their
  // weights are exactly 0 against the finite K and V of row 0.
  auto load = [&](const bf16_t* base, int kb, u32x4 (&rr)[8]) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int key = 32 * kb + 4 * r + (lane >> 4);
      rr[r] = ldw(base + (size_t)(key <= last ? key : 0) * HDIM + 8 * (lane & 15));
    }
  };
  auto stage = [&](const u32x4 (&rr)[8], int pitch) {
#pragma unroll
    for (int r = 0; r < 8; ++r) *reinterpret_cast<u32x4*>(&st[(4 * r + (lane >> 4)) * pitch + 8 * (lane & 15)]) = rr[r];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  };
  auto scores = [&](int kb, float (&sc)[16]) {
    // two independent 4-step MFMA chains (even and odd 16-dim steps), added at the end; Q^T
    // (query c, dims 16 kk + 8 hf ..) and K (key c, the same dims) from LDS, both with row pitch
    // QROW; the offset is opaque so the reads stay in the loop instead of being hoisted
    f32x16 acc, acc2;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = acc2[r] = 0.0f;
    int qo = c * QROW + 8 * hf;
    asm volatile("" : "+v"(qo));
    const bf16_t* qp = &sq[qo];
    const bf16_t* kp = &st[qo];
#pragma unroll
    for (int kk = 0; kk < 8; kk += 2) {
      const u32x4 q0 = *reinterpret_cast<const u32x4*>(qp + 16 * kk);
      const u32x4 q1 = *reinterpret_cast<const u32x4*>(qp + 16 * kk + 16);
      const u32x4 k0 = *reinterpret_cast<const u32x4*>(kp + 16 * kk);
      const u32x4 k1 = *reinterpret_cast<const u32x4*>(kp + 16 * kk + 16);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(k0), as_bf8(q0), acc, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(k1), as_bf8(q1), acc2, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] += acc2[r];
    // blocks that every query of the block sees whole (the wave-uniform common case) skip the mask
    if (32 * kb + 31 <= p0 + 32 * qb && 32 * qb + 31 < S) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = acc[r];
    } else {
      const int lim = qok ? qpos : -1;   // last key this lane's query sees (none past the prompt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * kb + 8 * (r >> 2) + 4 * hf + (r & 3);
        sc[r] = kr <= lim ? acc[r] : -INFINITY;
      }
    }
  };
  // e^(scale (s - m)) as 2^(s scale log2 e - m scale log2 e): one fma into the hardware exp2
  const float SL = scale * 1.4426950408889634f;
  auto ex = [SL](float s, float nm) { return __builtin_amdgcn_exp2f(fmaf(s, SL, nm)); };

  float m = -INFINITY, l = 0.0f;
  f32x16 o[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mb][r] = 0.0f;
  // transpose-read addresses of this lane (see above), relative to the staged V block
  const int gi = lane & 15, g = lane >> 4;
  const int tr_off = (4 * (g >> 1) + (gi >> 2)) * VROW + 16 * (g & 1) + 4 * (gi & 3);
  u32x4 kr[8], vr[8];
  // K before V here as in the loop: with the same load order on both edges into the loop, the
  // wait before each staging counts only the block it stages (the other block's prefetch stays in
  // flight); with V scheduled first here, the compiler waited for every load at the loop top
  load(kb_, w, kr);
  __builtin_amdgcn_sched_barrier(0);
  load(vb_, w, vr);
  for (int kb = w; kb < nkb; kb += AW) {
    stage(kr, QROW);
    load(kb_, kb + AW, kr);
    float sc[16];
    scores(kb, sc);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // K reads before the V staging
    stage(vr, VROW);
    load(vb_, kb + AW, vr);
    // running max; a fully masked row so far keeps m = -inf and adds nothing
    float bm = sc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) bm = fmaxf(bm, sc[r]);
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    const float nm = mn == -INFINITY ? 0.0f : -mn * SL;
    if (__builtin_amdgcn_ballot_w64(mn != m) != 0ull) {
      const float al = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m - mn) * SL);
      l *= al;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mb][r] *= al;
    }
    m = mn;
    float e[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      e[r] = ex(sc[r], nm);
      l += e[r];
    }
#pragma unroll
    for (int kk2 = 0; kk2 < 2; ++kk2) {
      u32x4 pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) pb[j] = pack_bh(e[8 * kk2 + 2 * j], e[8 * kk2 + 2 * j + 1]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16_t* vp = &st[16 * kk2 * VROW + 32 * mb + tr_off];
        const u32x2 lo = lds_tr16(vp);
        const u32x2 hi = lds_tr16(vp + 8 * VROW);
        const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
        o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(av), as_bf8(pb), o[mb], 0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // V reads before the next K staging
  }
  l += __shfl_xor(l, 32, 64);

  // merge the waves: M = max m_w, L = sum l_w e^(m_w - M), O = sum O_w e^(m_w - M) (wave order)
  __syncthreads();   // every wave's staging region is dead
  float* ob = reinterpret_cast<float*>(smem);
  float* sml = ob + (AW - 1) * HDIM * 32;   // [AW][2][32]
  if (hf == 0) {
    sml[(w * 2) * 32 + c] = m;
    sml[(w * 2 + 1) * 32 + c] = l;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int v = 0; v < AW; ++v) M = fmaxf(M, sml[(v * 2) * 32 + c]);
  const float sw = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m - M) * SL);
  if (w > 0) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) ob[((w - 1) * 64 + mb * 16 + r) * 64 + lane] = o[mb][r] * sw;
  }
  __syncthreads();
  if (w > 0 || !qok) return;
  float L = 0.0f;
#pragma unroll
  for (int v = 0; v < AW; ++v) {
    const float mv = sml[(v * 2) * 32 + c];
    L += mv == -INFINITY ? 0.0f : sml[(v * 2 + 1) * 32 + c] * __builtin_amdgcn_exp2f((mv - M) * SL);
  }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mb][r] *= sw;
#pragma unroll 1
  for (int v = 1; v < AW; ++v)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[mb][r] += ob[((v - 1) * 64 + mb * 16 + r) * 64 + lane];
  const float rl = L > 0.0f ? 1.0f / L : 0.0f;
  // O^T layout: column = query c, register r of block mb = dim 32 mb + 8 (r >> 2) + 4 hf + (r & 3)
  const size_t orow = (size_t)i * (NQH * HDIM) + hq * HDIM;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = 32 * mb + 8 * rq + 4 * hf;
      u32x2 pk;
      pk[0] = pack_bh(o[mb][4 * rq] * rl, o[mb][4 * rq + 1] * rl);
      pk[1] = pack_bh(o[mb][4 * rq + 2] * rl, o[mb][4 * rq + 3] * rl);
      *reinterpret_cast<u32x2*>(att + (frag ? frag_at(i, hq * HDIM + d0, NQH * HDIM) : orow + d0)) = pk;
    }
}

// First group-0 token from bf16 logits: ids [n-1024, n) except EOS suppressed when mask_tail
// (generator.py:71-75, :116), EOS suppressed when suppress_eos (min_new_tokens, :117-119), then
// the decode kernels' selection (greedy argmax, or temperature / top-k / top-p / Gumbel-max).
__global__ void __launch_bounds__(64) select_kernel(const bf16_t* logits, int n, int mask_tail, int eos_id,
                                                    int suppress_eos, SelParams sp, float* out_logits,
                                                    int* out_token) {
  __shared__ float stage[MAXV];
  __shared__ SelScratch sc;
  const int lane = threadIdx.x;
  // every logit load is issued before the first is used (a rolled loop waited for each in turn);
  // loads past n are clamped to n - 1 and dropped
  constexpr int NJ = (MAXV + 63) / 64;
  float lv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) lv[j] = bf2f(logits[min(lane + 64 * j, n - 1)]);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int i = lane + 64 * j;
    if (i >= n) break;
    float v = lv[j];
    if (out_logits) out_logits[i] = v;
    if (mask_tail && i >= n - 1024 && i != eos_id) v = -INFINITY;
    if (suppress_eos && i == eos_id) v = -INFINITY;
    stage[i] = v;
  }
  __syncthreads();
  const int tok = wave_select(stage, n, sp, &sc);
  if (lane == 0) *out_token = tok;
}

// ---- host ----------------------------------------------------------------------------------

struct Shape { int N, K; };
constexpr Shape kQKV{4096, HID}, kO{HID, NQH * HDIM}, kGU{2 * INTER, HID}, kDown{HID, INTER};

// tile width: 128 columns from 256 rows on (one LDS read per MFMA), 64 below (more tiles for
// the weight-streaming small-M case)
int tile_n(int M) { return M >= 256 ? 128 : 64; }

// split-K factor: double while the tile grid is below its target and the K range still splits
// into whole K steps. Targets: 128 workgroups below 256 rows (every split writes a full f32
// partial tile, which at 128 rows outweighs the weights it streams), one per CU from 256 rows.
// The SwiGLU GEMM is never split: its fused epilogue beats the unfused reduction at every M
// (measured at 128, 512 and 2048 rows), and its tile grid is the widest of the layer.
int splits_for(int M, int N, int K, bool swiglu = false) {
  if (swiglu) return 1;
  const int tn = tile_n(M), bk = tn == 64 ? bk_of<64>() : bk_of<128>();
  const int tiles = ((M + BM - 1) / BM) * (N / tn);
  const int target = M >= 256 ? 256 : 128;
  int ks = 1;
  while (tiles * ks < target && ks < MAX_SPLIT && (K / bk) % (2 * ks) == 0) ks *= 2;
  return ks;
}

// The row GEMM (M <= RM) per projection: tile width and split count, for a grid of 192-256
// workgroups (QKV 128 tiles x 2 splits, O and down 32 tiles x 8, gate/up 192 tiles unsplit)
constexpr int rows_tn(int) { return 32; }
constexpr int rows_ks(int wm) { return wm == W_QKV ? 2 : (wm == W_GU ? 1 : 8); }
constexpr Shape shape_of(int wm) { return wm == W_QKV ? kQKV : (wm == W_O ? kO : (wm == W_GU ? kGU : kDown)); }
int splits_of(int wm, int M) {
  const Shape sh = shape_of(wm);
  return M <= RM ? rows_ks(wm) : splits_for(M, sh.N, sh.K, wm == W_GU);
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Layout {
  size_t h, xn, qkv, att, act, hb, logits, part, total;
};

Layout layout(int S, int vocab) {
  Layout L;
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
  L.h = take((size_t)S * HID * 2);
  // the row GEMM's token operands hold whole 16-row blocks
  const size_t SP = S <= RM ? (size_t)(S + 15) / 16 * 16 : (size_t)S;
  L.xn = take(SP * HID * 2);
  L.qkv = take((size_t)S * QKVW * 2);
  L.att = take(SP * NQH * HDIM * 2);
  L.act = take(SP * INTER * 2);
  L.hb = take(HID * 2);
  L.logits = take((size_t)(vocab > 0 ? vocab : MAXV) * 2);
  size_t pb = 0;
  for (int wm : {W_QKV, W_O, W_DOWN}) {
    const int ks = splits_of(wm, S);
    if (ks > 1) pb = std::max(pb, (size_t)ks * S * shape_of(wm).N * 4);
  }
  const int ksh = splits_for(1, vocab > 0 ? vocab : MAXV, HID);
  if (ksh > 1) pb = std::max(pb, (size_t)ksh * (vocab > 0 ? vocab : MAXV) * 4);
  L.part = take(pb);
  L.total = o;
  return L;
}

template <int WM, int EPI, int TN>
void gemm_launch(const GemmArgs& g, int ks, bool reduce, hipStream_t st) {
  dim3 grid(g.N / TN, (g.M + BM - 1) / BM, ks);
  hipLaunchKernelGGL((gemm_kernel<WM, EPI, TN>), grid, dim3(GT), 0, st, g);
  if (ks > 1 && reduce) {
    const long nout = (long)g.M * (EPI == E_SWIGLU ? g.N / 2 : g.N) / 4;
    hipLaunchKernelGGL((reduce_kernel<EPI, TN>), dim3((unsigned)((nout + 255) / 256)), dim3(256), 0, st, g, ks);
  }
}

// Launches the GEMM; with split-K the partial sums are left in g.part for a fused consumer when
// `reduce` is false, else reduced here. `rope` (QKV only): an unsplit 128-column QKV GEMM finishes
// the heads itself (q/k-norm, RoPE, K/V write). Returns the split count (0 on a launch error).
template <int WM, int EPI>
int gemm(GemmArgs& g, hipStream_t st, bool reduce = true, const RopeArgs* rope = nullptr) {
  if constexpr (WM != W_DIRECT) {
    if (g.M <= RM) {
      constexpr int TN = rows_tn(WM), KS = rows_ks(WM), K = shape_of(WM).K;
      static_assert(K % (KS * 128) == 0 && (KS == 1 || EPI != E_SWIGLU), "row GEMM plan");
      if (g.K != K || g.N != shape_of(WM).N) return 0;
      g.kchunk = K / KS;
      hipLaunchKernelGGL((gemm_rows_kernel<WM, EPI, TN, K / KS / 128>), dim3(g.N / TN, 1, KS), dim3(GT), 0, st, g);
      if (KS > 1 && reduce)
        hipLaunchKernelGGL((reduce_kernel<EPI, 64>), dim3((unsigned)(((long)g.M * g.N / 4 + 255) / 256)), dim3(256), 0,
                           st, g, KS);
      return hipGetLastError() == hipSuccess ? KS : 0;
    }
  }
  const int ks = splits_for(g.M, g.N, g.K, EPI == E_SWIGLU);
  g.kchunk = g.K / ks;
  if (tile_n(g.M) == 128) {
    // two stages and two workgroups per CU when the grid covers the CUs twice or more; a grid of
    // at most one workgroup per CU (the split O and down projections) takes three stages instead
    const dim3 grid(g.N / 128, (g.M + 127) / 128, ks);
    const RopeArgs rr = (rope != nullptr && ks == 1) ? *rope : RopeArgs{};
    if (grid.x * grid.y * grid.z > 256)
      hipLaunchKernelGGL((gemm_dma_kernel<WM, EPI, 2>), grid, dim3(GT), 0, st, g, rr);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<WM, EPI, 3>), grid, dim3(GT), 0, st, g, rr);
    if (ks > 1 && reduce) {
      const long nout = (long)g.M * (EPI == E_SWIGLU ? g.N / 2 : g.N) / 4;
      hipLaunchKernelGGL((reduce_kernel<EPI, 128>), dim3((unsigned)((nout + 255) / 256)), dim3(256), 0, st, g, ks);
    }
  } else {
    gemm_launch<WM, EPI, 64>(g, ks, reduce, st);
  }
  return hipGetLastError() == hipSuccess ? ks : 0;
}

}  // namespace pf
}  // namespace qtts

using namespace qtts;
using namespace qtts::pf;

extern "C" {

size_t qtts_prefill_workspace_bytes(int n_tokens, int vocab) {
  if (n_tokens < 1 || vocab < 0 || vocab > MAXV) return 0;
  return layout(n_tokens, vocab).total;
}

hipError_t qtts_backbone_prefill(void* workspace, size_t workspace_bytes, const TTSLayerWeights* layer_weights,
                                 int num_layers, const void* final_norm_weight, const void* cos_table,
                                 const void* sin_table, void* k_cache, void* v_cache, int max_seq_len, int position,
                                 int n_tokens, const int* pos3, const void* input_embeddings, float* out_hidden,
                                 const void* codec_head, int vocab, float* out_logits, int* out_token, int mask_tail,
                                 int eos_id, int suppress_eos, const QttsSampling* sampling, int frame_step,
                                 hipStream_t stream) {
  const int S = n_tokens;
  if (workspace == nullptr || layer_weights == nullptr || final_norm_weight == nullptr || cos_table == nullptr ||
      sin_table == nullptr || k_cache == nullptr || v_cache == nullptr || input_embeddings == nullptr)
    return hipErrorInvalidValue;
  if (num_layers < 1 || S < 1 || position < 0 || max_seq_len < 1 || position + S > max_seq_len)
    return hipErrorInvalidValue;
  if (codec_head != nullptr && (vocab < 128 || vocab > MAXV || vocab % 128 != 0 || out_token == nullptr))
    return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0 || (reinterpret_cast<uintptr_t>(input_embeddings) & 15u) != 0)
    return hipErrorInvalidValue;
  const Layout L = layout(S, codec_head ? vocab : 0);
  if (workspace_bytes < L.total) return hipErrorInvalidValue;
  char* ws = static_cast<char*>(workspace);
  bf16_t* h = reinterpret_cast<bf16_t*>(ws + L.h);
  bf16_t* xn = reinterpret_cast<bf16_t*>(ws + L.xn);
  bf16_t* qkv = reinterpret_cast<bf16_t*>(ws + L.qkv);
  bf16_t* att = reinterpret_cast<bf16_t*>(ws + L.att);
  bf16_t* act = reinterpret_cast<bf16_t*>(ws + L.act);
  bf16_t* hb = reinterpret_cast<bf16_t*>(ws + L.hb);
  float* part = reinterpret_cast<float*>(ws + L.part);
  auto* kc = static_cast<bf16_t*>(k_cache);
  auto* vc = static_cast<bf16_t*>(v_cache);
  const auto* cs = static_cast<const bf16_t*>(cos_table);
  const auto* sn = static_cast<const bf16_t*>(sin_table);
  const float scale = 1.0f / sqrtf((float)HDIM);
  const unsigned norm_grid = (unsigned)((S + 3) / 4);
  // prompts the row GEMM takes: its token operands (xn, att, act) in the token-fragment layout
  const int frag = S <= RM ? 1 : 0;

  hipError_t e = hipMemcpyAsync(h, input_embeddings, (size_t)S * HID * 2, hipMemcpyDeviceToDevice, stream);
  if (e != hipSuccess) return e;
  // layer 0's input norm; later input norms come with the previous layer's down projection
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(norm_grid), dim3(256), 0, stream, h, HID, layer_weights, 0, 0,
                     (const bf16_t*)nullptr, xn, HID, (float*)nullptr, S, frag);
  const unsigned rows = (unsigned)S;
  const RopeArgs rope{cs, sn, pos3, position, kc, vc, max_seq_len};
  for (int l = 0; l < num_layers; ++l) {
    GemmArgs g{};
    g.layers = layer_weights;
    g.layer = l;
    g.M = S;
    g.part = part;
    int ks;
    // QKV, then q/k-norm + RoPE + K/V write: in the GEMM's epilogue (unsplit 128-column tiles), in
    // the split-K reduction, or (64-column tiles, unsplit) in rope_kv_kernel
    g.A = xn; g.lda = HID; g.N = kQKV.N; g.K = kQKV.K; g.out = qkv; g.ldo = QKVW;
    if ((ks = gemm<W_QKV, E_STORE>(g, stream, false, &rope)) == 0) return hipGetLastError();
    if (ks == 1 && tile_n(S) == 128) {
      // q/k-norm, RoPE and the K/V write ran in the QKV GEMM's epilogue
    } else if (ks > 1)
      hipLaunchKernelGGL(reduce_rope_kernel, dim3(rows), dim3(256), 0, stream, g, ks, cs, sn, pos3, position, kc, vc,
                         max_seq_len);
    else
      hipLaunchKernelGGL(rope_kv_kernel, dim3(rows), dim3(256), 0, stream, qkv, layer_weights, l, cs, sn, pos3, position,
                         S, kc, vc, max_seq_len);
    hipLaunchKernelGGL(attn_kernel, dim3((S + 31) / 32 * NQH), dim3(64 * AW), 0, stream, qkv, kc, vc, l, max_seq_len,
                       position, S, att, scale, frag);
    // O + residual, then the post-attention norm (fused with the split-K reduction)
    g.A = att; g.lda = NQH * HDIM; g.N = kO.N; g.K = kO.K; g.out = h; g.ldo = HID; g.res = h; g.ldr = HID;
    if ((ks = gemm<W_O, E_RESID>(g, stream, false)) == 0) return hipGetLastError();
    if (ks > 1)
      hipLaunchKernelGGL(reduce_resid_norm_kernel, dim3(rows), dim3(256), 0, stream, g, ks, l, 7, xn, frag);
    else
      hipLaunchKernelGGL(rmsnorm_kernel, dim3(norm_grid), dim3(256), 0, stream, h, HID, layer_weights, l, 7,
                         (const bf16_t*)nullptr, xn, HID, (float*)nullptr, S, frag);
    g.A = xn; g.lda = HID; g.N = kGU.N; g.K = kGU.K; g.out = act; g.ldo = INTER; g.res = nullptr;
    if (gemm<W_GU, E_SWIGLU>(g, stream) == 0) return hipGetLastError();
    // down + residual, then the next layer's input norm (fused with the split-K reduction)
    const int nl = l + 1 < num_layers ? l + 1 : -1;
    g.A = act; g.lda = INTER; g.N = kDown.N; g.K = kDown.K; g.out = h; g.ldo = HID; g.res = h; g.ldr = HID;
    if ((ks = gemm<W_DOWN, E_RESID>(g, stream, false)) == 0) return hipGetLastError();
    if (ks > 1)
      hipLaunchKernelGGL(reduce_resid_norm_kernel, dim3(rows), dim3(256), 0, stream, g, ks, nl, 0, xn, frag);
    else if (nl >= 0)
      hipLaunchKernelGGL(rmsnorm_kernel, dim3(norm_grid), dim3(256), 0, stream, h, HID, layer_weights, nl, 0,
                         (const bf16_t*)nullptr, xn, HID, (float*)nullptr, S, frag);
  }
  // final norm of the last token -> hidden (bf16 values; f32 copy for the caller)
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, stream, h + (size_t)(S - 1) * HID, HID,
                     (const TTSLayerWeights*)nullptr, 0, 0, static_cast<const bf16_t*>(final_norm_weight), hb, HID,
                     out_hidden, 1, 0);
  if (codec_head != nullptr) {
    bf16_t* lg = reinterpret_cast<bf16_t*>(ws + L.logits);
    GemmArgs g{};
    g.A = hb; g.lda = HID; g.B = static_cast<const bf16_t*>(codec_head); g.M = 1; g.N = vocab; g.K = HID;
    g.out = lg; g.ldo = vocab; g.part = part;
    if (gemm<W_DIRECT, E_STORE>(g, stream) == 0) return hipGetLastError();
    SelParams sp{};
    sp.do_sample = sampling ? sampling->do_sample : 0;
    sp.temperature = sampling ? sampling->temperature : 1.0f;
    sp.top_k = sampling ? sampling->top_k : 0;
    sp.top_p = sampling ? sampling->top_p : 1.0f;
    sp.seed = sampling ? sampling->seed : 0ull;
    sp.frame_step = frame_step;
    sp.group = 0;
    hipLaunchKernelGGL(select_kernel, dim3(1), dim3(64), 0, stream, lg, vocab, mask_tail, eos_id, suppress_eos, sp,
                       out_logits, out_token);
  }
  return hipGetLastError();
}

}  // extern "C"
