// Persistent decode kernels for Qwen3-TTS on MI355X (gfx950).
//
// Semantics follow the reference megakernels:
//   backbone:       /root/reference/qwentts_turbo/csrc/fused_decode_tts.cu:728-831
//   code predictor: /root/reference/qwentts_turbo/csrc/fused_decode_code_predictor.cu:565-668
// with the interleaved 3D mRoPE of rope_multimodal.cuh:9-54 (t, h, w may differ) and the
// frame glue of generator.py:116-174, 178-207, 309-362 moved on-device.
//
// Work decomposition (one launch of 256 workgroups, one per CU, all co-resident):
//   * Tensor-parallel over the 8 XCDs. XCD x owns KV head x with query heads 2x, 2x+1
//     (512 rows of Wq|Wk|Wv), intermediate rows [384x, 384x+384) of Wgate/Wup, and the
//     matching column slices of Wo ([:, 256x:256x+256]) and Wdown ([:, 384x:384x+384]).
//     Each XCD therefore produces a partial of the O and down projections; two cross-XCD
//     reductions per layer sum them (every XCD adds the 8 partials in the same order, so all
//     XCDs hold bit-identical activations).
//   * Inside an XCD the 32 workgroups split rows evenly: 16 QKV rows, 32 O rows, 12 gate +
//     12 up rows, 32 down rows each, so every weight byte is read exactly once per step.
//   * Attention of the XCD's KV head is split over C sequence chunks, one workgroup per
//     (chunk, query head); the poller of every O-projection workgroup merges the chunk partials
//     (m, l, acc). Contexts that fit one pass are attended locally by every workgroup.
//   * Each workgroup = 4 math waves + 1 poller wave. Math waves hold their weight slices in
//     VGPRs (the next step's tile issued one step ahead, the QKV, gate/up, down and head tiles
//     paced so that their HBM bursts spread over the exchanges in flight) and run the GEMVs and
//     attention. The poller wave waits for the inputs of the next stage (tagged exchange slots,
//     see qtts_common.h), applies the vector work (RMSNorm, q/k-norm + RoPE, KV write, split-K
//     merge, the cross-XCD sums + residuals, token selection) and leaves ready operands in LDS. Keeping
//     the polls on their own wave keeps them out of the math waves' in-order load queue.
#include <hip/hip_runtime.h>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>
#include "qtts_common.h"
#include "qtts_host.h"
#include "qtts_poll.h"
#include "qtts_select.h"
#include "qwentts_amd.h"

namespace qtts {

// Forced inlining for the step lambdas the compiler would otherwise call (their one-stream-per-XCD
// branches make them large): a real call passes the by-value launch arguments by address, which
// copies them to scratch memory.
#define QTTS_INLINE __attribute__((always_inline))

// ---------------------------------------------------------------------------------------
// Workspace (device): exchange slots, double-buffered by layer-pass parity.
// ---------------------------------------------------------------------------------------
struct Workspace {
  uint64_t qkv[NXCD][2][LROWS];
  uint64_t attp[NXCD][2][MAXC * APS];
  uint64_t h1[NXCD][2][HID];
  uint64_t inter[NXCD][2][XI];
  uint64_t xl[NXCD][2][HID];
  uint64_t opart[2][NXCD][HID];
  uint64_t dpart[2][NXCD][HID];
  uint64_t logits[2][MAXV];
  // greedy heads, two-level candidate exchange ({value, tag, index, tag} each):
  //   hloc: each math wave's best (4 per workgroup), read by the 32 workgroups of its XCD
  //   hx:   every workgroup's copy of its XCD's best, [li][xcd], read by the 8 workgroups li
  uint64_t hloc[NXCD][2][2 * NMATH * WPX];
  uint64_t hx[2][WPX][2 * NXCD];
  uint32_t err;
  uint32_t pad[63];
};

enum TagSlot { T_QKV = 0, T_ATT, T_OPART, T_H1, T_INTER, T_DPART, T_XL, T_NSLOT = 8 };
constexpr uint32_t TAG_HEAD = 3584;   // head logits tags: TAG_HEAD + position index
constexpr int MAX_LAYER_PASSES = 440; // layer passes per launch: 8 * 440 < TAG_HEAD

// Per-stream launch arguments. A batch-1 launch fills io[0]; a launch with one stream per XCD
// fills io[x] for the stream of XCD x.
constexpr int NSTREAM = NXCD;
struct StreamIO {
  Workspace* ws;
  void* kc;
  void* vc;
  int pos0;        // cache slot of the first position
  int pos3[3];     // rotary (t, h, w) of a single backbone position
  const bf16_t* in_emb;    // bf16 [1024] input of the first position
  int in_tok;              // token-id gather when in_emb == nullptr
  float* out_hidden;       // f32 [1024] final-norm hidden
  void* out_residual;      // bf16 (backbone) / f32 (CP) [1024], may be null
  float* out_logits;
  int* out_token;
  const int* history;
  int n_history;
  const int* skip;
  // code-predictor frame
  const float* bb_hidden;
  const int* g0;
  const bf16_t* text_row;
  int* out_tokens;
  int* hist_slot;
  bf16_t* out_combined;
  int* done;
  uint64_t seed;           // sampler key
};

// Per-launch arguments (passed by value).
struct KArgs {
  const TTSLayerWeights* layers;
  int num_layers;
  const bf16_t* final_norm;
  const bf16_t* cos_t;
  const bf16_t* sin_t;
  int max_seq;
  float scale;
  uint32_t tag_base;
  uint32_t spin_cap;
  uint32_t entry_spin_cap;   // cap of the first layer pass's waits (the arrival check)
  int n_pos;       // positions processed by this launch
  const bf16_t* embed_w;   // token-id gather table
  // backbone codec head + selection
  const bf16_t* head;
  int vocab;
  int mask_tail;
  float rep_penalty;
  int eos_id;
  int suppress_eos;
  // code-predictor frame
  int cp_frame;
  const bf16_t* bb_emb;
  const bf16_t* const* cp_heads;
  const bf16_t* const* cp_embs;
  int n_groups;
  int cp_vocab;
  SelParams sel;           // sampling parameters (the key is per stream)
  uint64_t* trace;         // optional step timeline: [wg][step][role] s_memrealtime stamps
  StreamIO io[NSTREAM];
};
constexpr int TRACE_STEPS = 1024;

// LDS of one workgroup.
// Arrays the math waves read sit in the first 64 KB, so their LDS accesses use one base
// register plus an immediate offset (the ds_* offset field is 16 bits); poller-only buffers
// and the selection scratch follow.
struct Lds {
  union {
    double red[NMATH][2][8][64];   // chunked attention partials [wave][head][dim % 8][lane group * 16 + dim / 8]
    struct {
      float vst[16][HDIM];         // code-predictor local attention: V of the context positions
      // code-predictor frame, two-column pass: the operands of position 1 (column 1; position
      // 0 uses the arrays below)
      alignas(16) float xn_1[HID];
      alignas(16) float hn_1[HID];
      alignas(16) float inter_1[XI];
      alignas(16) float q_1[2][HDIM];
      alignas(16) float knew_1[HDIM];
      alignas(16) float vnew_1[HDIM];
      alignas(16) float attn_1[2 * HDIM];
    };
  };
  double pl[2][16];                // (unused by the f32 code-predictor attention; kept for layout)
  alignas(16) float plf[2][16];    // code-predictor local attention: p_j = exp(s_j - M) per head
  float redmf[NMATH][2];           // its per-wave score maxima
  double redl[NMATH][4][2];         // their softmax sums
  double redm[2][NMATH][2];         // per (pass parity, wave, head) score max
  double wts[2][MAXC + 1];          // per head: chunk weights exp(m_c - M), then 1 / Z
  alignas(16) float q[2][HDIM];
  alignas(16) float knew[HDIM];
  alignas(16) float vnew[HDIM];
  alignas(16) float attn[2 * HDIM];    // attention output of the XCD's two heads
  alignas(16) float xn[HID];
  alignas(16) float hn[HID];
  float inter[XI];
  alignas(16) float hb[HID];
  // poller-only from here
  alignas(16) float xres[HID];
  alignas(16) float h1res[HID];
  alignas(16) float xres_1[HID];   // two-column pass: position 1's residual stream
  alignas(16) float h1res_1[HID];
  alignas(16) float comb[HID];   // code-predictor frame (workgroup 0): running embedding combine
  alignas(16) float stage[MAXV];
  uint32_t pen_bits[MAXV / 32];
  int tok[32];
  const bf16_t* embp[16];   // code-predictor embedding tables, loaded once per launch
  SelScratch sel;
};

// ---------------------------------------------------------------------------------------
// Math-wave register tiles
// ---------------------------------------------------------------------------------------
struct TileQKV { u32x4 p[8]; };
struct TileO { u32x4 p[4]; };
struct TileGU { u32x4 g[6]; u32x4 u[6]; };
struct TileD { u32x4 p[6]; };

enum { W_LNIN = 0, W_Q, W_K, W_V, W_QN, W_KN, W_O, W_LNPOST, W_GATE, W_UP, W_DOWN };
__device__ __forceinline__ const bf16_t* lw(const TTSLayerWeights* layers, int layer, int i) {
  const void* const* p = reinterpret_cast<const void* const*>(layers + layer);
  return reinterpret_cast<const bf16_t*>(ld_const(p + i));
}

// KV geometry. bf16 cache (backbone): a position is 16 pieces of 8 dims; per wave 16
// positions = 4 steps (jj) of 4 positions (one per 16-lane group). f32 cache (code predictor):
// a position is 32 pieces of 4 dims; per wave 4 positions (one per 16-lane group), each lane
// holding 2 pieces (8 dims). SUB = positions one pass of the 4 math waves covers (a whole
// code-predictor frame context, L <= 16, in one pass); CSUB = the chunking granularity for
// longer contexts (a chunk per CSUB positions, at most MAXC chunks).
template <bool BB> struct KVGeo;
template <> struct KVGeo<true> { static constexpr int JJ = 4, PPP = 1, SUB = 64, CSUB = 64; };
template <> struct KVGeo<false> { static constexpr int JJ = 1, PPP = 2, SUB = 16, CSUB = 2; };
// Column of the code-predictor frame's two-column pass (positions 0 and 1 share one pass over
// the weights): Col0 = position 0 (and every single-column step), Col1 = position 1.
using Col0 = std::integral_constant<int, 0>;
using Col1 = std::integral_constant<int, 1>;

template <bool BB> struct TileKV {
  u32x4 k[KVGeo<BB>::JJ * KVGeo<BB>::PPP];
  u32x4 v[KVGeo<BB>::JJ * KVGeo<BB>::PPP];
};

template <bool BB>
__device__ __forceinline__ void chunking(int L, int& C, int& P) {
  constexpr int CSUB = KVGeo<BB>::CSUB;
  int c0 = (L + CSUB - 1) / CSUB;
  if (c0 > MAXC) c0 = MAXC;
  if (c0 < 1) c0 = 1;
  P = (L + c0 - 1) / c0;
  C = (L + P - 1) / P;
}

template <bool BB>
__device__ __forceinline__ u32x4 wload(const bf16_t* p) {
  if constexpr (BB) return ldw_nt(p); else return ldw(p);
}

// The QKV tile. SLEEP > 0 paces it one row (two loads per lane) at a time, SLEEP x 64 cycles apart: the
// code predictor issues it after its down partials are published (or after a head), and whole, its 8.4 MB
// burst lands on the down all-reduce's cross-XCD hop (SLEEP 12, ~0.4 us: frame 920 -> 902 us; 8 apart
// 919 us, halves 32 or 48 apart slower). With the down tile paced too, SLEEP 16 at every site: frame
// 892 -> 885 us (20 apart: 894 us, 24: 889 us). The backbone's QKV tile is slower paced (16: +2 us).
template <bool BB, int SLEEP = 0>
__device__ __forceinline__ void load_qkv(TileQKV& t, const TTSLayerWeights* L, int layer, int xcd, int li, int mw, int lane) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int lr = 16 * li + 4 * mw + r;   // local row of the XCD's 512
    const bf16_t* row;
    if (lr < 256) row = lw(L, layer, W_Q) + (size_t)(256 * xcd + lr) * HID;
    else if (lr < 384) row = lw(L, layer, W_K) + (size_t)(128 * xcd + lr - 256) * HID;
    else row = lw(L, layer, W_V) + (size_t)(128 * xcd + lr - 384) * HID;
    t.p[2 * r] = wload<BB>(row + 8 * lane);
    t.p[2 * r + 1] = wload<BB>(row + 512 + 8 * lane);
    if constexpr (SLEEP > 0) {
      if (r < 3) __builtin_amdgcn_s_sleep(SLEEP);
    }
  }
}
template <bool BB>
__device__ __forceinline__ void load_o(TileO& t, const TTSLayerWeights* L, int layer, int xcd, int li, int mw, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 32 * li + 8 * mw + 2 * j + (lane >> 5);
    t.p[j] = wload<BB>(lw(L, layer, W_O) + (size_t)row * (NQH * HDIM) + 256 * xcd + 8 * (lane & 31));
  }
}
template <bool BB>
__device__ __forceinline__ void load_gu(TileGU& t, const TTSLayerWeights* L, int layer, int xcd, int li, int mw, int lane) {
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const size_t row = (size_t)(XI * xcd + 12 * li + 3 * mw + r) * HID;
    t.g[2 * r] = wload<BB>(lw(L, layer, W_GATE) + row + 8 * lane);
    t.g[2 * r + 1] = wload<BB>(lw(L, layer, W_GATE) + row + 512 + 8 * lane);
    t.u[2 * r] = wload<BB>(lw(L, layer, W_UP) + row + 8 * lane);
    t.u[2 * r + 1] = wload<BB>(lw(L, layer, W_UP) + row + 512 + 8 * lane);
  }
}
// Rows [R0, R1) of the wave's 3 gate/up row pairs (gate and up of each row).
template <bool BB, int R0, int R1>
__device__ __forceinline__ void load_gu_rows(TileGU& t, const TTSLayerWeights* L, int layer, int xcd, int li, int mw, int lane) {
#pragma unroll
  for (int r = R0; r < R1; ++r) {
    const size_t row = (size_t)(XI * xcd + 12 * li + 3 * mw + r) * HID;
    t.g[2 * r] = wload<BB>(lw(L, layer, W_GATE) + row + 8 * lane);
    t.g[2 * r + 1] = wload<BB>(lw(L, layer, W_GATE) + row + 512 + 8 * lane);
    t.u[2 * r] = wload<BB>(lw(L, layer, W_UP) + row + 8 * lane);
    t.u[2 * r + 1] = wload<BB>(lw(L, layer, W_UP) + row + 512 + 8 * lane);
  }
}
// One half of the gate/up tile: the gate rows (PART 0) or the up rows (PART 1).
template <bool BB, int PART>
__device__ __forceinline__ void load_gu_half(TileGU& t, const TTSLayerWeights* L, int layer, int xcd, int li, int mw, int lane) {
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const size_t row = (size_t)(XI * xcd + 12 * li + 3 * mw + r) * HID;
    if constexpr (PART == 0) {
      t.g[2 * r] = wload<BB>(lw(L, layer, W_GATE) + row + 8 * lane);
      t.g[2 * r + 1] = wload<BB>(lw(L, layer, W_GATE) + row + 512 + 8 * lane);
    } else {
      t.u[2 * r] = wload<BB>(lw(L, layer, W_UP) + row + 8 * lane);
      t.u[2 * r + 1] = wload<BB>(lw(L, layer, W_UP) + row + 512 + 8 * lane);
    }
  }
}
// The gate/up tile is the largest (12.6 MB over the GPU) and goes out right after the O partials are
// published, while the cross-XCD sums and then the h1 all-gather are in flight: issued whole, its HBM
// burst lands on the cross-XCD hop; deferred whole, on the all-gather. Paced instead, the two hops share
// it. Backbone: the gate rows, then the up rows 48 x 64 cycles (~1.5 us) later (step 493 -> 489 us).
// Code predictor: a third (one row pair) at a time, 24 x 64 cycles (~0.7 us) apart (frame 955 -> 915 us;
// halves 48 apart gave 926 us, thirds 16 apart 950 us, quarters 16 apart 919 us).
template <bool BB>
__device__ __forceinline__ void load_gu_paced(TileGU& t, const TTSLayerWeights* L, int layer, int xcd, int li, int mw, int lane) {
  if constexpr (BB) {
    load_gu_half<BB, 0>(t, L, layer, xcd, li, mw, lane);
    __builtin_amdgcn_s_sleep(48);
    load_gu_half<BB, 1>(t, L, layer, xcd, li, mw, lane);
  } else {
    load_gu_rows<BB, 0, 1>(t, L, layer, xcd, li, mw, lane);
    __builtin_amdgcn_s_sleep(24);
    load_gu_rows<BB, 1, 2>(t, L, layer, xcd, li, mw, lane);
    __builtin_amdgcn_s_sleep(24);
    load_gu_rows<BB, 2, 3>(t, L, layer, xcd, li, mw, lane);
  }
}
// The down tile: two row groups of 3 loads per lane, the second ~0.3 us (s_sleep 12) after the
// first, so that the burst does not all land on the SwiGLU all-gather. Code predictor: frame
// 898 -> 891 us (6 or 8 apart: 901 us, 16 apart: 894 us, 24 apart: 903 us, three pieces: 906 us);
// backbone: step 484.0 -> 482.4 us (16 apart: 482.4, 24 apart: 484.0).
template <bool BB, int SLEEP = 0>
__device__ __forceinline__ void load_d(TileD& t, const TTSLayerWeights* L, int layer, int xcd, int li, int mw, int lane) {
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int row = 32 * li + 8 * mw + 4 * g + (lane >> 4);
#pragma unroll
    for (int j = 0; j < 3; ++j)
      t.p[3 * g + j] = wload<BB>(lw(L, layer, W_DOWN) + (size_t)row * INTER + XI * xcd + 8 * ((lane & 15) + 16 * j));
    if constexpr (SLEEP > 0) { if (g == 0) __builtin_amdgcn_s_sleep(SLEEP); }
  }
}
// rows [row0 + 0 .. nrows) of a [*, 1024] head, nrows <= 3 per wave (into the QKV tile's registers).
// Non-temporal in both models: a code-predictor head (4 MB) is read once per frame, and kept out of the
// caches it leaves the 256 MB MALL to what is re-read sooner, the code predictor's layers (157 MB, 15 times
// per frame) and the backbone's KV cache (backbone step 486 -> 483 us at L=512). The code predictor's
// layer tiles stay temporal: non-temporal there, the frame went 900 -> 971 us (and the backbone 486 -> 472).
// SLEEP > 0: the rows after the first ~SLEEP x 64 cycles later (s_sleep 16 after a model's last down
// publish: frame 1,358.3 -> 1,356.1 us, code predictor and backbone together; 8 apart: 1,357.6).
template <bool BB, int SLEEP = 0>
__device__ __forceinline__ void load_head(TileQKV& t, const bf16_t* W, int row0, int nrows, int lane) {
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    if (r < nrows) {
      t.p[2 * r] = ldw_nt(W + (size_t)(row0 + r) * HID + 8 * lane);
      t.p[2 * r + 1] = ldw_nt(W + (size_t)(row0 + r) * HID + 512 + 8 * lane);
    }
    if constexpr (SLEEP > 0) { if (r == 0) __builtin_amdgcn_s_sleep(SLEEP); }
  }
}

// KV sub-block [b0, b0 + SUB) of the chunk, restricted to old positions (< min(bend, Lold)).
template <bool BB>
__device__ __forceinline__ void load_kv(TileKV<BB>& t, const KArgs& a, const void* kcp, const void* vcp, int layer, int kvh, int b0, int lim, int mw, int lane) {
  constexpr int JJ = KVGeo<BB>::JJ, PPP = KVGeo<BB>::PPP;
  const size_t head_base = ((size_t)layer * NKVH + kvh) * (size_t)a.max_seq;
#pragma unroll
  for (int jj = 0; jj < JJ; ++jj) {
    const int pos0_ = b0 + 4 * JJ * mw + 4 * jj + (lane >> 4);
    const bool ok = pos0_ < lim;
    const int pos = ok ? pos0_ : 0;   // every address stays inside the cache
#pragma unroll
    for (int pp = 0; pp < PPP; ++pp) {
      if constexpr (BB) {
        const size_t off = (head_base + (size_t)pos) * HDIM + 8 * (lane & 15);
        t.k[jj] = ok ? ldw(reinterpret_cast<const bf16_t*>(kcp) + off) : u32x4{0, 0, 0, 0};
        t.v[jj] = ok ? ldw(reinterpret_cast<const bf16_t*>(vcp) + off) : u32x4{0, 0, 0, 0};
      } else {
        // The code-predictor cache is rewritten inside one frame launch and read by other
        // CUs, so its loads are L2-coherent (sc1: no L1 line of an older write is used).
        // Lanes without a position read past the buffer end, which returns zeros.
        const uint32_t bytes = (uint32_t)((size_t)a.num_layers * NKVH * (size_t)a.max_seq * HDIM * 4);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(kcp), (short)0, (int)bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(vcp), (short)0, (int)bytes, 0x00020000);
        const uint32_t off = ok ? (uint32_t)(((head_base + (size_t)pos0_) * HDIM + 8 * (lane & 15) + 4 * pp) * 4) : 0xFFFFFFF0u;
        t.k[PPP * jj + pp] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 16);
        t.v[PPP * jj + pp] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 16);
      }
    }
  }
}
template <bool BB>
__device__ __forceinline__ void unpack8(const TileKV<BB>& t, bool key, int jj, float* o) {
  if constexpr (BB) {
    const u32x4 w = key ? t.k[jj] : t.v[jj];
    o[0] = bflo(w.x); o[1] = bfhi(w.x); o[2] = bflo(w.y); o[3] = bfhi(w.y);
    o[4] = bflo(w.z); o[5] = bfhi(w.z); o[6] = bflo(w.w); o[7] = bfhi(w.w);
  } else {
    const u32x4 w0 = key ? t.k[2 * jj] : t.v[2 * jj];
    const u32x4 w1 = key ? t.k[2 * jj + 1] : t.v[2 * jj + 1];
    o[0] = __uint_as_float(w0.x); o[1] = __uint_as_float(w0.y); o[2] = __uint_as_float(w0.z); o[3] = __uint_as_float(w0.w);
    o[4] = __uint_as_float(w1.x); o[5] = __uint_as_float(w1.y); o[6] = __uint_as_float(w1.z); o[7] = __uint_as_float(w1.w);
  }
}

// Sum of the 8 XCD partials of rows r0 + 2 (lane & 15) + {0, 1}: lane group g = lane >> 4 polls
// XCDs 2 g and 2 g + 1 and adds them; two exchanges (lane ^ 16, lane ^ 32) complete the sum as
// ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)), bit-identical in every lane and workgroup.
__device__ __forceinline__ bool poll_sum8(const Poll& P, const uint64_t (*part)[HID], int r0, uint32_t tag, double& s0, double& s1) {
  const uint32_t o = ws_off(P, &part[0][r0]);
  float v[4];
  const bool ok = poll_regs<2>(P, 128, tag, v, [o](int i) {
    const uint32_t x = 2u * (uint32_t)((i & 63) >> 4) + (uint32_t)(i >> 6);
    return o + x * (HID * 8u) + 16u * (uint32_t)(i & 15);
  });
  s0 = (double)v[0] + (double)v[2];
  s1 = (double)v[1] + (double)v[3];
  s0 += xlane_d<4>(s0);
  s1 += xlane_d<4>(s1);
  s0 += xlane_d<5>(s0);
  s1 += xlane_d<5>(s1);
  return ok;
}
// One stream per XCD: the 8 partials of rows r0 + 2 (lane + 64 k) + {0, 1} (k < 2, 256 rows) in
// this lane, summed as ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)), the order of poll_sum8.
// sum[2 k + j] is row r0 + 2 (lane + 64 k) + j.
__device__ __forceinline__ bool poll_sum8_rows(const Poll& P, const uint64_t (*part)[HID], int r0, uint32_t tag, double (&sum)[4]) {
  const uint32_t o = ws_off(P, &part[0][r0]);
  float v[32];
  const bool ok = poll_regs<16>(P, 1024, tag, v, [o](int i) {
    const uint32_t q = (uint32_t)i >> 6, l = (uint32_t)i & 63u;   // q = 8 k + x
    return o + (q & 7u) * (HID * 8u) + 16u * (l + 64u * (q >> 3));
  });
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      double p[NXCD];
#pragma unroll
      for (int x = 0; x < NXCD; ++x) p[x] = (double)v[2 * (8 * k + x) + j];
      sum[2 * k + j] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
  return ok;
}

// RMSNorm epsilon: the f32 constant 1e-6f of the reference, used in f64 arithmetic.
constexpr double EPSD = (double)1e-6f;


// ---------------------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------------------
// XL = one stream per XCD: stream x runs on the 32 workgroups of XCD x, which act as 8 virtual
// XCDs of 4 workgroups each (workgroup l of the XCD is virtual XCD l & 7 and takes its row groups
// 8 (l >> 3) .. 8 (l >> 3) + 7, one after another). The exchange slots and their order are those
// of the batch-1 decomposition, so every stream computes exactly what a batch-1 launch does.
template <bool BB, bool XL>
__global__ void __launch_bounds__(NTHR, 1) qtts_decode_kernel(const KArgs a) {
  __shared__ Lds s;
  // Accumulation type: f64 in the backbone (its bf16 residual and KV make every stored rounding
  // reproducible against the f64 oracle), f32 in the code predictor (f32 residual and KV, as
  // the reference's CP kernel computes them).
  using A = std::conditional_t<BB, double, float>;
  // lane index, re-derived opaquely at every step (see walk) so that lane-dependent slot
  // offsets are recomputed where used instead of being hoisted out of the step loop and
  // kept live (and spilled) across all steps
  int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool poller = wave == NMATH;
  const int mw = __builtin_amdgcn_readfirstlane(wave);   // wave-uniform: row bases stay in SGPRs
  const int xcd_hw = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u);  // HW_REG_XCC_ID
  const int li_hw = blockIdx.x >> 3;
  const int si = XL ? xcd_hw : 0;              // stream of this workgroup
  // this stream's block, read through the kernel-argument segment with a uniform offset (scalar
  // loads); indexing the by-value argument with a run-time index would copy it to scratch
  const __attribute__((address_space(4))) StreamIO* IO =
      (const __attribute__((address_space(4))) StreamIO*)((const __attribute__((address_space(4))) char*)
                                                          __builtin_amdgcn_kernarg_segment_ptr() + offsetof(KArgs, io)) + si;
  // per-stream field: XL through IO, batch 1 at its constant offset in the by-value arguments
#define SIO(f) (XL ? IO->f : a.io[0].f)
  const int xcd = XL ? (li_hw & 7) : xcd_hw;   // (virtual) XCD: KV head and row ownership
  const int li = XL ? 8 * (li_hw >> 3) : li_hw;  // first row group of this workgroup
  constexpr int NSUB = XL ? 8 : 1;             // row groups per workgroup
  const int wg = blockIdx.x;
  const bool lead = XL ? li_hw == 0 : wg == 0;   // the stream's lead workgroup
  Workspace* ws = SIO(ws);
  if (XL && ws == nullptr) return;   // no stream on this XCD

  if (SIO(skip) != nullptr && *SIO(skip) != 0) return;
  int g0 = 0;
  if (a.cp_frame) {
    g0 = *SIO(g0);
    if (a.eos_id >= 0 && g0 == a.eos_id) {
      if (lead && threadIdx.x == 0) *SIO(done) = 1;
      return;
    }
  }
  __syncthreads();

  Poll P;
  P.rs = __builtin_amdgcn_make_buffer_rsrc(ws, (short)0, (int)sizeof(Workspace), 0x00020000);
  P.base = ws;
  P.ec.err = &ws->err;
  // the first layer pass waits under the short entry cap (an arrival check: its exchanges need
  // every workgroup of the launch); the poller restores the long cap from the second pass on
  P.ec.spin_cap = a.entry_spin_cap;
  // Slot publishes go through the workspace buffer descriptor (SGPRs) with a 32-bit offset:
  // XCD-local slots as plain stores (they land in the XCD's L2), cross-XCD slots with sc1
  // (written through to memory). One 8-byte store carries value and tag together.
  auto pub_local = [&](const uint64_t* p, float v, uint32_t tag) {
    const u32x2 d = {__float_as_uint(v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(d, P.rs, (int)ws_off(P, p), 0, 0);
  };
  auto pub_cross = [&](const uint64_t* p, float v, uint32_t tag) {
    const u32x2 d = {__float_as_uint(v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(d, P.rs, (int)ws_off(P, p), 0, XL ? 0 : 16);   // XL: all in one XCD
  };
  const TTSLayerWeights* LW = a.layers;
  const int NL = a.num_layers;

  TileQKV tq;
  TileO to;
  TileGU tgu;
  TileD td;
  TileKV<BB> tk;

  auto tag_of = [&](int lp, int slot) -> uint32_t { return a.tag_base + (uint32_t)(lp * T_NSLOT + slot); };
  // greedy heads (code-predictor groups, the backbone's codec head) select through a two-level
  // exchange of workgroup candidates instead of gathering every logit in one workgroup
  const bool greedy_sel = !a.sel.do_sample && (BB || a.cp_frame);
  // backbone greedy head with a repetition penalty: the history as a bitmap in LDS (built at launch)
  const bool pen_rows = BB && !a.cp_frame && greedy_sel && a.head != nullptr && a.rep_penalty != 1.0f && SIO(n_history) > 0;
  auto has_head = [&](int pi) -> bool { return a.cp_frame ? pi >= 1 : (a.head != nullptr && pi == a.n_pos - 1); };

  // rotary row of channel c (c < 64) at position pos
  auto rot_row = [&](int c, int pos) -> int {
    if constexpr (BB) {
      const int sec = (c < 60 && c % 3 == 1) ? 1 : ((c < 60 && c % 3 == 2) ? 2 : 0);
      return a.n_pos == 1 ? SIO(pos3[sec]) : pos;
    } else {
      return pos;
    }
  };

  // ---- poller registers: small per-layer vectors, loaded a step (or a layer) before use so
  // that no dependent global load sits on the critical path of a step. The poller lane owns
  // hidden elements 2 (lane + 64 k) + {0, 1} (k < 8) and head channels lane, lane + 64 (the
  // rotate_half partners).
  //   g_in / g_post / g_fin: RMSNorm gains of the lane's 16 elements (8 packed bf16 pairs)
  //   qn / kn: q/k-norm gains of head channels lane, lane + 64; rc / rsn: their cos / sin
  uint32_t g_in[8], g_post[8], g_fin[8];
  float qn[2], kn[2], rc[2], rsn[2];
  // The next layer's gains are issued at the start of a step, before its poll, into these, and
  // take over at the step's end: the pointer-table read and the loads then overlap the wait
  // instead of sitting between the step's last vector work and the barrier.
  uint32_t g_in_n[8], g_post_n[8];
  float qn_n[2], kn_n[2], rc_n[2], rsn_n[2];
  float rc1[2], rsn1[2];   // two-column pass: rotary of position 1
  auto load_gain_pairs = [&](uint32_t (&g)[8], const bf16_t* src) {
    const auto* p = gmem(reinterpret_cast<const uint32_t*>(src));
#pragma unroll
    for (int k = 0; k < 8; ++k) g[k] = p[lane + 64 * k];
  };
  auto load_qk_gains_to = [&](int layer, float (&qd)[2], float (&kd)[2]) QTTS_INLINE {
    const bf16_t* q = lw(LW, layer, W_QN);
    const bf16_t* k = lw(LW, layer, W_KN);
    qd[0] = ldbf(q + lane); qd[1] = ldbf(q + lane + 64);
    kd[0] = ldbf(k + lane); kd[1] = ldbf(k + lane + 64);
  };
  auto load_qk_gains = [&](int layer) { load_qk_gains_to(layer, qn, kn); };
  auto take2 = [&](float (&d)[2], const float (&s2)[2]) QTTS_INLINE { d[0] = s2[0]; d[1] = s2[1]; };
  auto take8 = [&](uint32_t (&d)[8], const uint32_t (&s8)[8]) QTTS_INLINE {
#pragma unroll
    for (int k = 0; k < 8; ++k) d[k] = s8[k];
  };
  auto load_rope_to = [&](int pos, float (&c)[2], float (&sn)[2]) QTTS_INLINE {
    const size_t row = (size_t)rot_row(lane, pos) * HDIM;   // channel lane + 64 shares the row
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      c[j] = ldbf(a.cos_t + row + lane + 64 * j);
      sn[j] = ldbf(a.sin_t + row + lane + 64 * j);
    }
  };
  auto load_rope = [&](int pos) { load_rope_to(pos, rc, rsn); };
  // LDS operands of a column (Col0: the single-column arrays) and its exchange-buffer parity:
  // column 1 publishes with position 1's layer-pass tags into the parity buffer column 0 does
  // not use in the same step (by the exchange chain, every reader of a buffer is done before
  // the next step's writers reach it)
  constexpr bool DUO_OK = !BB && !XL;
  auto cxres = [&](auto c) QTTS_INLINE -> float* { if constexpr (decltype(c)::value == 1) return s.xres_1; else return s.xres; };
  auto cxn = [&](auto c) QTTS_INLINE -> float* { if constexpr (decltype(c)::value == 1) return s.xn_1; else return s.xn; };
  auto ch1res = [&](auto c) QTTS_INLINE -> float* { if constexpr (decltype(c)::value == 1) return s.h1res_1; else return s.h1res; };
  auto chn = [&](auto c) QTTS_INLINE -> float* { if constexpr (decltype(c)::value == 1) return s.hn_1; else return s.hn; };
  auto cinter = [&](auto c) QTTS_INLINE -> float* { if constexpr (decltype(c)::value == 1) return s.inter_1; else return s.inter; };
  auto cattn = [&](auto c) QTTS_INLINE -> float* { if constexpr (decltype(c)::value == 1) return s.attn_1; else return s.attn; };
  auto cpar = [&](int lp, auto c) QTTS_INLINE -> int {
    if constexpr (decltype(c)::value == 1) return ((lp - NL) & 1) ^ 1; else return lp & 1;
  };
  // RMSNorm statistic of the lane-distributed 1024-vector: 1 / sqrt(mean(x^2) + eps) in f64
  auto rstd_of = [&](const float (&xv)[16]) -> A {
    A s4[4] = {A(0), A(0), A(0), A(0)};
#pragma unroll
    for (int j = 0; j < 16; ++j) s4[j & 3] = fma((A)xv[j], (A)xv[j], s4[j & 3]);
    const A ss = group_sum<64>((s4[0] + s4[1]) + (s4[2] + s4[3]));
    return rsqrt_a(ss / (A)HID + (A)EPSD);
  };
  // normalized values f32((x * rstd) * g) of the lane's 16 elements
  // f64 copy of a gain slice, made before the step's poll (off the critical path)
  auto gains_d = [&](const uint32_t (&g)[8], A (&gd)[16]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) { gd[2 * k] = bflo(g[k]); gd[2 * k + 1] = bfhi(g[k]); }
  };
  auto normed = [&](const float (&xv)[16], const A (&gd)[16], float (&y)[16]) {
    const A r = rstd_of(xv);
#pragma unroll
    for (int j = 0; j < 16; ++j) y[j] = (float)(((A)xv[j] * r) * gd[j]);
  };
  auto store_pairs = [&](float* dst, const float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) *reinterpret_cast<float2*>(dst + 2 * (lane + 64 * k)) = make_float2(v[2 * k], v[2 * k + 1]);
  };
  // one 16-byte store of two adjacent XCD-local slots
  auto pub_local2 = [&](const uint64_t* p, float v0, float v1, uint32_t tag) {
    const u32x4 d = {__float_as_uint(v0), tag, __float_as_uint(v1), tag};
    __builtin_amdgcn_raw_buffer_store_b128(d, P.rs, (int)ws_off(P, p), 0, 0);
  };

  // ---- poller: input of layer 0 of position pi (embedding source) -> xres, xn
  auto prep_input0 = [&](int pi, auto col) QTTS_INLINE {
    A gd[16];
    gains_d(g_in, gd);
    float xv[16];
    if (a.cp_frame && pi == 0) {
      const auto* p = gmem(reinterpret_cast<const u32x2*>(SIO(bb_hidden)));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const u32x2 v = p[lane + 64 * k];
        xv[2 * k] = rbf(__uint_as_float(v.x));
        xv[2 * k + 1] = rbf(__uint_as_float(v.y));
      }
    } else {
      const bf16_t* src;
      if (a.cp_frame) src = pi == 1 ? a.bb_emb + (size_t)g0 * HID : s.embp[pi - 2] + (size_t)s.tok[pi - 2] * HID;
      else src = SIO(in_emb) != nullptr ? SIO(in_emb) : a.embed_w + (size_t)SIO(in_tok) * HID;
      const auto* p = gmem(reinterpret_cast<const uint32_t*>(src));
#pragma unroll
      for (int k = 0; k < 8; ++k) { const uint32_t w = p[lane + 64 * k]; xv[2 * k] = bflo(w); xv[2 * k + 1] = bfhi(w); }
    }
    store_pairs(cxres(col), xv);
    float y[16];
    normed(xv, gd, y);
    store_pairs(cxn(col), y);
  };

  // ---- poller (code-predictor frame, workgroup 0): the embedding combine, accumulated as each
  // position's input row arrives in xres (bf16 rounding after each add, in the order
  // emb_bb[g0] + emb_0[t_0] + emb_1[t_1] + ...; generator.py:356-362)
  auto comb_add = [&](bool first, auto col) QTTS_INLINE {
    const float* xr = cxres(col);
    for (int k = 0; k < 8; ++k) {
      const int e = 2 * (lane + 64 * k);
      const float2 x = *reinterpret_cast<const float2*>(&xr[e]);
      const float2 c = *reinterpret_cast<const float2*>(&s.comb[e]);
      *reinterpret_cast<float2*>(&s.comb[e]) = first ? x : make_float2(rbf(c.x + x.x), rbf(c.y + x.y));
    }
  };

  // ---- poller: AR2 of layer pass lp (down partials + residual) -> xl slots
  auto ar2 = [&](int lp, auto col) QTTS_INLINE {
    const int par = cpar(lp, col);
    const float* h1r = ch1res(col);
    if constexpr (XL) {
      // the workgroup's 8 row groups: rows 32 li + 2 (lane + 64 k) + {0, 1}
      double sm[4];
      float r[4];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        r[2 * k] = h1r[32 * li + 2 * (lane + 64 * k)];
        r[2 * k + 1] = h1r[32 * li + 2 * (lane + 64 * k) + 1];
      }
      poll_sum8_rows(P, ws->dpart[par], 32 * li, tag_of(lp, T_DPART), sm);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        float x0 = (float)((double)r[2 * k] + sm[2 * k]), x1 = (float)((double)r[2 * k + 1] + sm[2 * k + 1]);
        if constexpr (BB) { x0 = rbf(x0); x1 = rbf(x1); }
        pub_local2(&ws->xl[xcd][par][32 * li + 2 * (lane + 64 * k)], x0, x1, tag_of(lp, T_XL));
      }
      return;
    }
    const int row = 32 * li + 2 * (lane & 15);
    const float r0 = h1r[row], r1 = h1r[row + 1];
    double s0, s1;
    poll_sum8(P, ws->dpart[par], 32 * li, tag_of(lp, T_DPART), s0, s1);
    if (lane < 16) {
      // x' = h1 + the sum of the 8 XCD partials, in f64
      float x0 = (float)((double)r0 + s0), x1 = (float)((double)r1 + s1);
      if constexpr (BB) { x0 = rbf(x0); x1 = rbf(x1); }
      pub_local2(&ws->xl[xcd][par][row], x0, x1, tag_of(lp, T_XL));
    }
  };
  // ---- poller: next layer input (after ar2 of lp) -> xres, xn
  auto prep_input_next = [&](int lp, auto col) QTTS_INLINE {
    float xv[16], y[16];
    A gd[16];
    gains_d(g_in, gd);
    poll_vec_regs(P, ws->xl[xcd][cpar(lp, col)], tag_of(lp, T_XL), xv);
    store_pairs(cxres(col), xv);
    normed(xv, gd, y);
    store_pairs(cxn(col), y);
  };
  // ---- poller: final norm (after ar2 of lp) -> hb (bf16-rounded), outputs
  auto prep_final = [&](int lp, auto col) QTTS_INLINE {
    float xv[16], y[16];
    A gd[16];
    gains_d(g_fin, gd);
    poll_vec_regs(P, ws->xl[xcd][cpar(lp, col)], tag_of(lp, T_XL), xv);
    store_pairs(s.xres, xv);
    normed(xv, gd, y);
    if (lead) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = 2 * (lane + 64 * k);
        if (SIO(out_hidden)) *reinterpret_cast<float2*>(SIO(out_hidden) + e) = make_float2(y[2 * k], y[2 * k + 1]);
        if (SIO(out_residual)) {
          if constexpr (BB)
            reinterpret_cast<uint32_t*>(SIO(out_residual))[e >> 1] =
                (uint32_t)f2bf(xv[2 * k]) | ((uint32_t)f2bf(xv[2 * k + 1]) << 16);
          else
            *reinterpret_cast<float2*>(reinterpret_cast<float*>(SIO(out_residual)) + e) = make_float2(xv[2 * k], xv[2 * k + 1]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) y[j] = rbf(y[j]);
    store_pairs(s.hb, y);
  };
  // ---- poller: q/k norm, RoPE, KV write for layer `layer` at position pos
  // The lane holds channels c = lane and c + 64 (the rotate_half partners) of q head 0, q head 1,
  // k and v (the QKV slot order pairs them).
  bool kv_pending = false;
  // The KV entry of the new token is read only by workgroups of this XCD (KV head = XCD), at
  // later positions, through this XCD's L2 (L1-bypassing loads). Its stores reaching L2 before
  // this wave's next slot publish is therefore all the ordering needed: a wait for the wave's
  // outstanding vector stores, not an agent-scope release (whose L2 write-back would sit on
  // the critical path of every layer).
  auto kv_write_done = [&]() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  auto prep_att = [&](int lp, int layer, int pos, int C, auto col) QTTS_INLINE {
    constexpr bool c1 = decltype(col)::value == 1;
    const int par = cpar(lp, col);
    const A cl = c1 ? rc1[0] : rc[0], ch = c1 ? rc1[1] : rc[1], sl = c1 ? rsn1[0] : rsn[0], sh = c1 ? rsn1[1] : rsn[1];
    float (&sq)[2][HDIM] = c1 ? s.q_1 : s.q;
    float* skn = c1 ? s.knew_1 : s.knew;
    float* svn = c1 ? s.vnew_1 : s.vnew;
    float v[8];   // [head][j]: head 0, 1 = q, 2 = k, 3 = v; j = 0: channel c, 1: channel c + 64
    {
      const uint32_t o = ws_off(P, ws->qkv[xcd][par]);
      poll_regs<4>(P, LROWS / 2, tag_of(lp, T_QKV), v, [o](int i) { return o + 16u * (uint32_t)i; });
    }
    A ss[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) ss[h] = fma((A)v[2 * h], (A)v[2 * h], (A)v[2 * h + 1] * (A)v[2 * h + 1]);
    group_sum_n<64, 3>(ss);
    float outl[3], outh[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      const A r = rsqrt_a(ss[h] / (A)HDIM + (A)EPSD);
      const A gl = h < 2 ? qn[0] : kn[0], gh = h < 2 ? qn[1] : kn[1];
      const A nl = ((A)v[2 * h] * r) * gl, nh = ((A)v[2 * h + 1] * r) * gh;
      outl[h] = (float)(nl * cl - nh * sl);
      outh[h] = (float)(nl * sh + nh * ch);
    }
    const int c = lane;
    sq[0][c] = outl[0]; sq[0][c + 64] = outh[0];
    sq[1][c] = outl[1]; sq[1][c + 64] = outh[1];
    float kl = outl[2], kh = outh[2], vl = v[6], vh = v[7];
    if constexpr (BB) { kl = rbf(kl); kh = rbf(kh); vl = rbf(vl); vh = rbf(vh); }
    skn[c] = kl; skn[c + 64] = kh;
    svn[c] = vl; svn[c + 64] = vh;
    if (C - 1 >= li && C - 1 < li + NSUB) {
      const size_t off = (((size_t)layer * NKVH + xcd) * (size_t)a.max_seq + pos) * HDIM + c;
      if constexpr (BB) {
        bf16_t* kc = reinterpret_cast<bf16_t*>(SIO(kc)) + off;
        bf16_t* vc = reinterpret_cast<bf16_t*>(SIO(vc)) + off;
        gput(kc, f2bf(kl)); gput(kc + 64, f2bf(kh));
        gput(vc, f2bf(vl)); gput(vc + 64, f2bf(vh));
      } else {
        float* kc = reinterpret_cast<float*>(SIO(kc)) + off;
        float* vc = reinterpret_cast<float*>(SIO(vc)) + off;
        gput(kc, kl); gput(kc + 64, kh);
        gput(vc, vl); gput(vc + 64, vh);
      }
      // ordered before this wave's next slot publish (prep_gu), where the wait for the stores
      // costs nothing: the entry is read only at later positions or launches
      kv_pending = true;
    }
  };
  // ---- poller: merge the 2C attention partials (chunk c, head h) of the XCD's KV head into
  // s.attn (the split-K combine of fused_decode_tts.cu:282-385). Every unit's (m, l) pair, one
  // 16-byte slot pair per unit (lane (h, c); lanes past C re-read chunk C - 1): per head the
  // chunk weights w_c = exp(m_c - M), M = max_c m_c, and Z = sum_c l_c w_c, over the 16 chunk
  // lanes with four exchanges. Lane (h, j) takes dims 4j .. 4j + 3 of every chunk of head h and
  // merges them in f64: f32((sum_c acc_c w_c) * (1 / Z)). The (m, l) pairs and the first HC
  // chunks' accumulators come in one poll; the accumulators of chunks HC.. (contexts beyond
  // HC chunks) in a second read, once the first has seen every unit's (m, l) (they have about
  // landed by then; the registers of one poll of all 16 would spill).
  auto prep_o = [&](int lp, int C) {
    constexpr int HC = MAXC / 2;
    const int par = lp & 1;
    const uint32_t o = ws_off(P, ws->attp[xcd][par]);
    const uint32_t tg = tag_of(lp, T_ATT);
    const int h = lane >> 5, c = lane & 31;
    // k = 0 the (m, l) pair of unit (chunk c, head h), k = 1 + 2 cc + e the acc dims
    // 4 (lane & 31) + 2 e, +1 of chunk cc, head h
    auto off = [o, C](int i, int cbase) {
      const uint32_t k = (uint32_t)i >> 6, l = (uint32_t)i & 63u;
      if (k == 0u) {
        const int cc = min((int)(l & 31u), C - 1);
        return o + 8u * (uint32_t)((2 * cc + (int)(l >> 5)) * APH + 128);
      }
      const uint32_t kk = k - 1u, cc = (uint32_t)cbase + (kk >> 1);
      return o + 8u * ((2u * cc + (l >> 5)) * (uint32_t)APH + 4u * (l & 31u) + 2u * (kk & 1u));
    };
    float v[2 + 4 * HC];
    poll_regs<1 + 2 * HC>(P, 64 * (1 + 2 * min(C, HC)), tg, v, [off](int i) { return off(i, 0); });
    {
      const bool ok = c < C;
      const float mc = ok ? v[0] : -INFINITY;
      const float lc = ok ? v[1] : 0.0f;
      float M = mc;
      M = fmaxf(M, xlane_f<0>(M));
      M = fmaxf(M, xlane_f<1>(M));
      M = fmaxf(M, xlane_f<2>(M));
      M = fmaxf(M, xlane_f<3>(M));
      const double w = ok ? exp((double)mc - (double)M) : 0.0;
      double Z = (double)lc * w;
      Z += xlane_d<0>(Z);
      Z += xlane_d<1>(Z);
      Z += xlane_d<2>(Z);
      Z += xlane_d<3>(Z);
      if (c < MAXC) s.wts[h][c] = w;
      if (c == 0) s.wts[h][MAXC] = 1.0 / Z;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");   // the weights written above
    double a4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int cc = 0; cc < HC; ++cc) {
      if (cc < C) {   // chunks past C were not polled (their registers hold no value)
        const double w = s.wts[h][cc];
#pragma unroll
        for (int j = 0; j < 4; ++j) a4[j] = fma((double)v[2 + 4 * cc + j], w, a4[j]);
      }
    }
    if (C > HC) {
      float u[4 * HC];
      read_pairs<2 * HC>(P, 64 * 2 * (C - HC), tg, u, [off](int i) { return off(i + 64, HC); });
#pragma unroll
      for (int cc = 0; cc < HC; ++cc) {
        if (HC + cc < C) {
          const double w = s.wts[h][HC + cc];
#pragma unroll
          for (int j = 0; j < 4; ++j) a4[j] = fma((double)u[4 * cc + j], w, a4[j]);
        }
      }
    }
    const double rz = s.wts[h][MAXC];
    *reinterpret_cast<float4*>(&s.attn[128 * h + 4 * c]) =
        make_float4((float)(a4[0] * rz), (float)(a4[1] * rz), (float)(a4[2] * rz), (float)(a4[3] * rz));
  };
  // ---- poller: AR1 (O partials + residual) -> h1 slots; then h1 -> h1res, hn
  auto ar1 = [&](int lp, auto col) QTTS_INLINE {
    const int par = cpar(lp, col);
    const float* xr = cxres(col);
    // h1 = x + the sum of the 8 XCD partials, in f64
    if constexpr (XL) {
      double sm[4];
      float r[4];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        r[2 * k] = xr[32 * li + 2 * (lane + 64 * k)];
        r[2 * k + 1] = xr[32 * li + 2 * (lane + 64 * k) + 1];
      }
      poll_sum8_rows(P, ws->opart[par], 32 * li, tag_of(lp, T_OPART), sm);
      if (kv_pending) {
        kv_write_done();   // the KV entry written in prep_att
        kv_pending = false;
      }
#pragma unroll
      for (int k = 0; k < 2; ++k)
        pub_local2(&ws->h1[xcd][par][32 * li + 2 * (lane + 64 * k)], (float)((double)r[2 * k] + sm[2 * k]),
                   (float)((double)r[2 * k + 1] + sm[2 * k + 1]), tag_of(lp, T_H1));
    } else {
      const int row = 32 * li + 2 * (lane & 15);
      const float r0 = xr[row], r1 = xr[row + 1];
      double s0, s1;
      poll_sum8(P, ws->opart[par], 32 * li, tag_of(lp, T_OPART), s0, s1);
      if (kv_pending) {
        kv_write_done();   // the KV entry written in prep_att
        kv_pending = false;
      }
      if (lane < 16) pub_local2(&ws->h1[xcd][par][row], (float)((double)r0 + s0), (float)((double)r1 + s1), tag_of(lp, T_H1));
    }
  };
  // h1 gathered -> h1res, hn
  auto gather_h1 = [&](int lp, auto col) QTTS_INLINE {
    float xv[16], y[16];
    A gd[16];
    gains_d(g_post, gd);
    poll_vec_regs(P, ws->h1[xcd][cpar(lp, col)], tag_of(lp, T_H1), xv);
    store_pairs(ch1res(col), xv);
    normed(xv, gd, y);
    store_pairs(chn(col), y);
  };
  auto prep_gu = [&](int lp, int layer, auto col) QTTS_INLINE {
    ar1(lp, col);
    gather_h1(lp, col);
  };
  auto prep_down = [&](int lp, auto col) QTTS_INLINE {
    poll_vec<3>(P, ws->inter[xcd][cpar(lp, col)], XI, tag_of(lp, T_INTER), cinter(col));
  };

  // ---- math: attention over this workgroup's chunk [c0, c1) at KV length L, for NH query
  // heads: both heads of the XCD's KV head (NH = 2, one pass over the K/V tile serves both),
  // or head hh alone (NH = 1: the chunked split gives each (chunk, head) its own workgroup).
  // Lane group g (16 lanes x 8 dims) scores positions b0 + 4 JJ mw + 4 jj + g (jj < JJ); the
  // workgroup shares one running max per head, so lane-group partials are plain sums: they go
  // to LDS unscaled and thread (head, dim) adds them. Every exp is branch-free (a masked
  // argument becomes -1000, whose exp is 0).
  auto attention = [&](auto nh_c, int lp, int layer, int L, int c0, int c1, bool local, int hh, int unit) {
    constexpr int NH = decltype(nh_c)::value;
    constexpr int JJ = KVGeo<BB>::JJ, SUB = KVGeo<BB>::SUB;
    constexpr double NEG = -1000.0;
    const int Lold = L - 1;
    const int d0 = 8 * (lane & 15), g = lane >> 4;
    const double scale = (double)a.scale;
    const int nsb = (c1 - c0 + SUB - 1) / SUB;
    const int hq0 = NH == 2 ? 0 : hh;   // first query head of this workgroup
    double qv[NH][8];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[h][i] = s.q[hq0 + h][d0 + i];
    double m[NH], l[NH], acc[NH][8];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      m[h] = -INFINITY;
      l[h] = 0.0;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] = 0.0;
    }
    for (int sb = 0; sb < nsb; ++sb) {
      const int b0 = c0 + sb * SUB;
      if (sb > 0) load_kv<BB>(tk, a, SIO(kc), SIO(vc), layer, xcd, b0, c1 < Lold ? c1 : Lold, mw, lane);
      double sc[NH * JJ];
#pragma unroll
      for (int jj = 0; jj < JJ; ++jj) {
        const int pos = b0 + 4 * JJ * mw + 4 * jj + g;
        float kv[8];
        if (pos == Lold) {
#pragma unroll
          for (int i = 0; i < 8; ++i) kv[i] = s.knew[d0 + i];
        } else {
          unpack8<BB>(tk, true, jj, kv);
        }
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          double dd = 0.0;
#pragma unroll
          for (int i = 0; i < 8; ++i) dd = fma(qv[h][i], (double)kv[i], dd);
          sc[h * JJ + jj] = dd;
        }
      }
      group_sum_n<16>(sc);
      // f32-rounded scores; masked positions -inf; wave-wide max per head
      double mx[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        double mloc = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < JJ; ++jj) {
          const int pos = b0 + 4 * JJ * mw + 4 * jj + g;
          const double v = pos < c1 ? (double)(float)(sc[h * JJ + jj] * scale) : -INFINITY;
          sc[h * JJ + jj] = v;
          mloc = v > mloc ? v : mloc;
        }
        double u = xlane_d<4>(mloc);
        mloc = u > mloc ? u : mloc;
        u = xlane_d<5>(mloc);
        mx[h] = u > mloc ? u : mloc;
      }
      // workgroup-wide maximum of this pass (slots double-buffered by pass parity): every
      // wave and lane group then shares one running max, so their partial sums add plainly
      if (lane == 0) {
#pragma unroll
        for (int h = 0; h < NH; ++h) s.redm[sb & 1][mw][h] = mx[h];
      }
      step_barrier();
      double mn[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        double M = m[h];
#pragma unroll
        for (int w = 0; w < NMATH; ++w) M = s.redm[sb & 1][w][h] > M ? s.redm[sb & 1][w][h] : M;
        mn[h] = M;
      }
      if (sb > 0) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const double alpha = exp(m[h] == -INFINITY ? NEG : m[h] - mn[h]);
          l[h] *= alpha;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[h][i] *= alpha;
        }
      }
      double pr[NH * JJ];
      if constexpr (NH * JJ % 4 == 0) {
        // every lane of a 16-lane group holds all NH * JJ scores: lane l exponentiates those with
        // k = l (mod 4) and its quad shares them (one f64 exp per lane instead of NH * JJ)
        const int q4 = opaque((int)threadIdx.x) & 3;
#pragma unroll
        for (int k4 = 0; k4 < NH * JJ / 4; ++k4) {
          double arg = NEG;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int k = 4 * k4 + j;
            const double v = sc[k] == -INFINITY ? NEG : sc[k] - mn[k / JJ];
            arg = q4 == j ? v : arg;
          }
          const double e = exp(arg);
          pr[4 * k4 + 0] = quad_bcast_d<0>(e);
          pr[4 * k4 + 1] = quad_bcast_d<1>(e);
          pr[4 * k4 + 2] = quad_bcast_d<2>(e);
          pr[4 * k4 + 3] = quad_bcast_d<3>(e);
        }
      } else {
#pragma unroll
        for (int k = 0; k < NH * JJ; ++k) pr[k] = exp(sc[k] == -INFINITY ? NEG : sc[k] - mn[k / JJ]);
      }
#pragma unroll
      for (int jj = 0; jj < JJ; ++jj) {
        const int pos = b0 + 4 * JJ * mw + 4 * jj + g;
        float vv[8];
        if (pos == Lold) {
#pragma unroll
          for (int i = 0; i < 8; ++i) vv[i] = s.vnew[d0 + i];
        } else {
          unpack8<BB>(tk, false, jj, vv);
        }
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          l[h] += pr[h * JJ + jj];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[h][i] = fma(pr[h * JJ + jj], (double)vv[i], acc[h][i]);
        }
      }
#pragma unroll
      for (int h = 0; h < NH; ++h) m[h] = mn[h];
    }
    // the wave's softmax sums (its 4 lane groups), one value per head; partials lane-major (each
    // store of the wave writes 64 consecutive doubles: no bank conflicts)
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      l[h] += xlane_d<4>(l[h]);
      l[h] += xlane_d<5>(l[h]);
#pragma unroll
      for (int i = 0; i < 8; ++i) s.red[mw][h][i][lane] = acc[h][i];
      if (lane == 0) s.redl[mw][0][h] = l[h];
    }
    step_barrier();
    // thread t merges dim d = 8 j + i of head h, reading row i at columns 16 g + j (contiguous in j)
    const int t = threadIdx.x;  // 0..255
    const int h = t >> 7, ii = (t >> 4) & 7, jj0 = t & 15, d = 8 * jj0 + ii;
    if (h < NH) {
      double A = 0.0, Lsum = 0.0;
#pragma unroll
      for (int w = 0; w < NMATH; ++w) {
        A += (s.red[w][h][ii][jj0] + s.red[w][h][ii][16 + jj0]) + (s.red[w][h][ii][32 + jj0] + s.red[w][h][ii][48 + jj0]);
        Lsum += s.redl[w][0][h];
      }
      if (local) {
        // the whole context in this workgroup: f32(A * (1 / l)), no partial exchange
        s.attn[128 * (hq0 + h) + d] = (float)(A * (1.0 / Lsum));
      } else {
        // partial of (chunk unit >> 1, head hh = unit & 1): acc[128], m, l
        uint64_t* dst = &ws->attp[xcd][lp & 1][unit * APH];
        const uint32_t tg = tag_of(lp, T_ATT);
        pub_local(dst + d, (float)A, tg);
        if (d == 0) { pub_local(dst + 128, (float)m[0], tg); pub_local(dst + 129, (float)Lsum, tg); }
      }
    }
    step_barrier();   // s.red is reused by the next attention; s.attn complete
  };

  // ---- math: code-predictor attention over the whole context (L <= 16), in f32. Lane group g of
  // math wave w takes position j = 4 w + g: its score per head (8 dims per lane, summed over
  // the 16 lanes), the wave maximum, then after one barrier the workgroup maximum M and
  // p_j = exp(s_j - M); p and V_j go to LDS and, after a second barrier, thread (h, d) forms
  // (sum_j p_j V_j[d]) / (sum_j p_j) from operands it loads all at once. Positions j >= L carry
  // p = 0 and V = 0 (the tile's out-of-range lanes read zeros), so the sums run over all 16.
  // duo (two-column pass, L = 2): position 1 (column 1) attends to positions 0 and 1, both new
  // entries in LDS; position 0 (column 0) attends to itself alone, whose result is its V exactly
  // (p = exp(0) = 1, Z = 1), stored directly.
  auto attention_cp_local = [&](int L, auto duo_c) QTTS_INLINE {
    constexpr bool duo = decltype(duo_c)::value;
    const int Lold = L - 1;
    const int d0 = 8 * (lane & 15), g = lane >> 4;
    const int j = 4 * mw + g;
    float kv[8], vv[8];
    const float (&sq)[2][HDIM] = duo ? s.q_1 : s.q;
    const float4 qa0 = *reinterpret_cast<const float4*>(&sq[0][d0]), qb0 = *reinterpret_cast<const float4*>(&sq[0][d0 + 4]);
    const float4 qa1 = *reinterpret_cast<const float4*>(&sq[1][d0]), qb1 = *reinterpret_cast<const float4*>(&sq[1][d0 + 4]);
    if (duo) {
      // j = 0: position 0's entry; j = 1: position 1's; positions past L carry zeros
      const float* ks = j == 0 ? s.knew : s.knew_1;
      const float* vs = j == 0 ? s.vnew : s.vnew_1;
      const bool ok = j < 2;
      const float4 ka = ok ? *reinterpret_cast<const float4*>(&ks[d0]) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 kb = ok ? *reinterpret_cast<const float4*>(&ks[d0 + 4]) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 va = ok ? *reinterpret_cast<const float4*>(&vs[d0]) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 vb = ok ? *reinterpret_cast<const float4*>(&vs[d0 + 4]) : make_float4(0.f, 0.f, 0.f, 0.f);
      kv[0] = ka.x; kv[1] = ka.y; kv[2] = ka.z; kv[3] = ka.w; kv[4] = kb.x; kv[5] = kb.y; kv[6] = kb.z; kv[7] = kb.w;
      vv[0] = va.x; vv[1] = va.y; vv[2] = va.z; vv[3] = va.w; vv[4] = vb.x; vv[5] = vb.y; vv[6] = vb.z; vv[7] = vb.w;
    } else if (j == Lold) {
      const float4 ka = *reinterpret_cast<const float4*>(&s.knew[d0]), kb = *reinterpret_cast<const float4*>(&s.knew[d0 + 4]);
      const float4 va = *reinterpret_cast<const float4*>(&s.vnew[d0]), vb = *reinterpret_cast<const float4*>(&s.vnew[d0 + 4]);
      kv[0] = ka.x; kv[1] = ka.y; kv[2] = ka.z; kv[3] = ka.w; kv[4] = kb.x; kv[5] = kb.y; kv[6] = kb.z; kv[7] = kb.w;
      vv[0] = va.x; vv[1] = va.y; vv[2] = va.z; vv[3] = va.w; vv[4] = vb.x; vv[5] = vb.y; vv[6] = vb.z; vv[7] = vb.w;
    } else {
      unpack8<BB>(tk, true, 0, kv);
      unpack8<BB>(tk, false, 0, vv);
    }
    const float q0[8] = {qa0.x, qa0.y, qa0.z, qa0.w, qb0.x, qb0.y, qb0.z, qb0.w};
    const float q1[8] = {qa1.x, qa1.y, qa1.z, qa1.w, qb1.x, qb1.y, qb1.z, qb1.w};
    float sc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sc[0] = fmaf(q0[i], kv[i], sc[0]);
      sc[1] = fmaf(q1[i], kv[i], sc[1]);
    }
    group_sum_n<16>(sc);
    float mx[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[h] = j < L ? sc[h] * a.scale : -INFINITY;
      mx[h] = fmaxf(sc[h], xlane_f<4>(sc[h]));
      mx[h] = fmaxf(mx[h], xlane_f<5>(mx[h]));
    }
    if (lane == 0) { s.redmf[mw][0] = mx[0]; s.redmf[mw][1] = mx[1]; }
    // V of this lane's position, staged for the weighted sums (read after the second barrier)
    *reinterpret_cast<float4*>(&s.vst[j][d0]) = make_float4(vv[0], vv[1], vv[2], vv[3]);
    *reinterpret_cast<float4*>(&s.vst[j][d0 + 4]) = make_float4(vv[4], vv[5], vv[6], vv[7]);
    step_barrier();
    float p[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float M = fmaxf(fmaxf(s.redmf[0][h], s.redmf[1][h]), fmaxf(s.redmf[2][h], s.redmf[3][h]));
      p[h] = j < L ? __expf(sc[h] - M) : 0.0f;
    }
    if ((lane & 15) == 0) { s.plf[0][j] = p[0]; s.plf[1][j] = p[1]; }
    step_barrier();
    const int t = threadIdx.x;   // 0..255: head t >> 7, dim t & 127
    const int h = t >> 7, d = t & 127;
    float pj[16], vj[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 pp = *reinterpret_cast<const float4*>(&s.plf[h][4 * q]);
      pj[4 * q] = pp.x; pj[4 * q + 1] = pp.y; pj[4 * q + 2] = pp.z; pj[4 * q + 3] = pp.w;
    }
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) vj[jj] = s.vst[jj][d];
    // four independent chains (positions jj = 4 i + c), combined at the end
    float A4[4] = {0.0f, 0.0f, 0.0f, 0.0f}, Z4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      Z4[jj & 3] += pj[jj];
      A4[jj & 3] = fmaf(pj[jj], vj[jj], A4[jj & 3]);
    }
    const float As = (A4[0] + A4[1]) + (A4[2] + A4[3]), Z = (Z4[0] + Z4[1]) + (Z4[2] + Z4[3]);
    if (duo) {
      s.attn_1[t] = As * rcp_f(Z);
      s.attn[t] = s.vnew[d];
    } else {
      s.attn[t] = As * rcp_f(Z);
    }
    step_barrier();   // s.attn complete; vst / plf are reused by the next attention
  };

  // ---- math: GEMV stages (f64 accumulation, f32 results)
  auto load_x16 = [&](const float* x, A* xv) {
#pragma unroll
    for (int i = 0; i < 8; ++i) { xv[i] = x[8 * lane + i]; xv[8 + i] = x[512 + 8 * lane + i]; }
  };
  auto math_qkv = [&](int lp, int lg, const TileQKV& tq, auto col) QTTS_INLINE {
    A xv[16];
    load_x16(cxn(col), xv);
    const uint32_t tg = tag_of(lp, T_QKV);
    A v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = dot8a(tq.p[2 * r + 1], xv + 8, dot8a(tq.p[2 * r], xv, A(0)));
    const A t = rs_sum<5, 4>(v, lane);   // row lane >> 4 in lanes 0, 16, 32, 48
    // slot order pairs the rotate_half partners: channel c' of head h goes to slot
    // 128 h + 2 (c' mod 64) + c' / 64, so one 16-byte pair holds channels c and c + 64
    const int lr = 16 * lg + 4 * mw + (lane >> 4), cc = lr & 127;
    if ((lane & 15) == 0) pub_local(&ws->qkv[xcd][cpar(lp, col)][(lr & ~127) + 2 * (cc & 63) + (cc >> 6)], (float)t, tg);
  };
  auto math_o = [&](int lp, int lg, const TileO& to, auto colc) QTTS_INLINE {
    const int col = 8 * (lane & 31);
    const float* at = cattn(colc);
    A xv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = at[col + i];
    const uint32_t tg = tag_of(lp, T_OPART);
    A v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = dot8a(to.p[j], xv, A(0));
    // per half-wave: row pair j = (lane >> 3) & 3 ends in lanes 0, 8, 16, 24 (+32)
    const A t = rs_sum<4, 4>(v, lane);
    if ((lane & 7) == 0)
      pub_cross(&ws->opart[cpar(lp, colc)][xcd][32 * lg + 8 * mw + 2 * ((lane >> 3) & 3) + (lane >> 5)], (float)t, tg);
  };
  auto math_gu = [&](int lp, int lg, const TileGU& tgu, auto col) QTTS_INLINE {
    A xv[16];
    load_x16(chn(col), xv);
    const uint32_t tg = tag_of(lp, T_INTER);
    using P2 = pair2<A>;
    P2 c[4];
#pragma unroll
    for (int r = 0; r < 3; ++r)
      c[r] = P2{dot8a(tgu.g[2 * r + 1], xv + 8, dot8a(tgu.g[2 * r], xv, A(0))),
                dot8a(tgu.u[2 * r + 1], xv + 8, dot8a(tgu.u[2 * r], xv, A(0)))};
    c[3] = P2{A(0), A(0)};
    const P2 t = rs_sum<5, 4>(c, lane);   // (gate, up) of row lane >> 4 in lanes 0, 16, 32
    const int r = lane >> 4;
    if ((lane & 15) == 0 && r < 3) {
      const A act = t.a / (A(1) + exp_a(-t.a)) * t.b;
      pub_local(&ws->inter[xcd][cpar(lp, col)][12 * lg + 3 * mw + r], (float)act, tg);
    }
  };
  auto math_down = [&](int lp, int lg, const TileD& td, auto col) QTTS_INLINE {
    const float* it = cinter(col);
    A xv[24];
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[8 * j + i] = it[8 * ((lane & 15) + 16 * j) + i];
    const uint32_t tg = tag_of(lp, T_DPART);
    A v[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      v[g] = A(0);
#pragma unroll
      for (int j = 0; j < 3; ++j) v[g] = dot8a(td.p[3 * g + j], xv + 8 * j, v[g]);
    }
    // per 16-lane group: row set g = (lane >> 3) & 1 ends in lanes 0 and 8
    const A t = rs_sum<3, 2>(v, lane);
    if ((lane & 7) == 0)
      pub_cross(&ws->dpart[cpar(lp, col)][xcd][32 * lg + 8 * mw + 4 * ((lane >> 3) & 1) + (lane >> 4)], (float)t, tg);
  };
  // head rows of a workgroup (of its row group sub in XL): backbone codec head 12 rows (3 per
  // wave), CP head 8 (2 per wave)
  auto head_rows = [&](int sub, int& row0, int& nrows) {
    const int per_wg = (a.cp_frame ? a.cp_vocab : a.vocab) / NWG;
    nrows = per_wg / NMATH;
    row0 = (XL ? 8 * li_hw + sub : wg) * per_wg + mw * nrows;
  };
  // head logits of row group sub from tile tq: greedy code-predictor heads fold them into the
  // wave's best (bv, bi) (larger value, lowest id on ties); the other heads publish them
  auto head_group = [&](int pi, int sub, const TileQKV& tq, float& bv, int& bi) {
    int row0, nrows;
    head_rows(sub, row0, nrows);
    A xv[16];
    load_x16(s.hb, xv);
    const uint32_t tg = a.tag_base + TAG_HEAD + (uint32_t)pi;
    A v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      v[r] = r < 3 && r < nrows ? dot8a(tq.p[2 * r + 1], xv + 8, dot8a(tq.p[2 * r], xv, A(0))) : A(0);
    const A t = rs_sum<5, 4>(v, lane);   // row lane >> 4 in lanes 0, 16, 32, 48
    const int r = lane >> 4;
    // logits are bf16 values, as the reference's torch.mv over bf16 operands returns them
    // (generator.py:158, :351); ties then go to the lowest id, as torch.argmax
    if (greedy_sel) {
      const int ci0 = row0 + r;
      float cv = -INFINITY;
      if ((lane & 15) == 0 && r < nrows) {
        cv = rbf((float)t);
        if (BB && !a.cp_frame) {
          // the backbone's codec head: raw logit out, then the selection's mask, repetition
          // penalty and EOS suppression on this row (generator.py:71-75, 161-167)
          if (SIO(out_logits)) SIO(out_logits[ci0]) = cv;
          if (a.mask_tail && ci0 >= a.vocab - 1024 && ci0 != a.eos_id) cv = -INFINITY;
          if (pen_rows && ((s.pen_bits[ci0 >> 5] >> (ci0 & 31)) & 1u)) cv = rbf(cv > 0.f ? cv / a.rep_penalty : cv * a.rep_penalty);
          if (a.suppress_eos && ci0 == a.eos_id) cv = -INFINITY;
        }
      }
      int ci = ci0;
      best_merge(cv, ci, xlane_f<4>(cv), (int)xlane<4>((uint32_t)ci));
      best_merge(cv, ci, xlane_f<5>(cv), (int)xlane<5>((uint32_t)ci));
      best_merge(bv, bi, cv, ci);
    } else if ((lane & 15) == 0 && r < nrows) {
      const float lv = rbf((float)t);
      pub_cross(&ws->logits[pi & 1][row0 + r], lv, tg);
      if (!a.cp_frame && SIO(out_logits)) SIO(out_logits[row0 + r]) = lv;
    }
  };
  // greedy code-predictor head: only the workgroup's best (value, lowest id on ties) is published;
  // the selecting waves reduce the workgroup candidates instead of the whole vocabulary
  // (each math wave publishes its own best: no workgroup barrier on the way to the exchange)
  auto head_publish = [&](int pi, float bv, int bi) {
    if (!greedy_sel) return;
    const uint32_t tg = a.tag_base + TAG_HEAD + (uint32_t)pi;
    if (lane == 0) {
      const u32x4 d = {__float_as_uint(bv), tg, (uint32_t)bi, tg};
      const int slot = NMATH * (XL ? li_hw : li) + mw;
      __builtin_amdgcn_raw_buffer_store_b128(d, P.rs, (int)ws_off(P, &ws->hloc[XL ? 0 : xcd][pi & 1][2 * slot]), 0, 0);
    }
  };
  auto head_weights = [&](int pi) -> const bf16_t* {
    return a.cp_frame ? ld_const(a.cp_heads + (pi - 1)) : a.head;
  };
  // ---- poller: collect a head's logits and select a token
  auto select = [&](int pi) -> int {
    if (greedy_sel) {
      // Candidates {value, index} are merged by larger value, lower index on ties (an
      // order-independent choice). Level 1: the 128 wave bests of this XCD (L2-local), two per lane.
      const uint32_t tg = a.tag_base + TAG_HEAD + (uint32_t)pi;
      const int par = pi & 1;
      float cv[4];
      {
        const uint32_t o = ws_off(P, &ws->hloc[XL ? 0 : xcd][par][0]);
        poll_regs<2>(P, NMATH * WPX, tg, cv, [o](int i) { return o + 16u * (uint32_t)i; });
      }
      float bv = cv[0];
      int bi = (int)__float_as_uint(cv[1]);
      best_merge(bv, bi, cv[2], (int)__float_as_uint(cv[3]));
#pragma unroll
      for (int st = 0; st < 6; ++st) {
        float ov;
        int oi;
        switch (st) {
          case 0: ov = xlane_f<0>(bv); oi = (int)xlane<0>((uint32_t)bi); break;
          case 1: ov = xlane_f<1>(bv); oi = (int)xlane<1>((uint32_t)bi); break;
          case 2: ov = xlane_f<2>(bv); oi = (int)xlane<2>((uint32_t)bi); break;
          case 3: ov = xlane_f<3>(bv); oi = (int)xlane<3>((uint32_t)bi); break;
          case 4: ov = xlane_f<4>(bv); oi = (int)xlane<4>((uint32_t)bi); break;
          default: ov = xlane_f<5>(bv); oi = (int)xlane<5>((uint32_t)bi); break;
        }
        best_merge(bv, bi, ov, oi);
      }
      if constexpr (XL) {
        // one stream per XCD: the XCD's best is the stream's
        bi = __builtin_amdgcn_readfirstlane(bi);
        return (bi >= 0 && bi < (a.cp_frame ? a.cp_vocab : a.vocab)) ? bi : 0;
      }
      // Level 2: this workgroup's copy of the XCD best goes to hx[li][xcd]; the 8 XCD bests are
      // read from the copies of workgroup index li (each cache line has 8 readers).
      if (lane == 0) {
        const u32x4 d = {__float_as_uint(bv), tg, (uint32_t)bi, tg};
        __builtin_amdgcn_raw_buffer_store_b128(d, P.rs, (int)ws_off(P, &ws->hx[par][li][2 * xcd]), 0, 16);
      }
      float cx[2];
      {
        const uint32_t o = ws_off(P, &ws->hx[par][li][0]);
        poll_regs<1>(P, NXCD, tg, cx, [o](int i) { return o + 16u * (uint32_t)i; });
      }
      bv = lane < NXCD ? cx[0] : -INFINITY;
      bi = lane < NXCD ? (int)__float_as_uint(cx[1]) : 0x7fffffff;
#pragma unroll
      for (int st = 0; st < 3; ++st) {
        float ov;
        int oi;
        switch (st) {
          case 0: ov = xlane_f<0>(bv); oi = (int)xlane<0>((uint32_t)bi); break;
          case 1: ov = xlane_f<1>(bv); oi = (int)xlane<1>((uint32_t)bi); break;
          default: ov = xlane_f<2>(bv); oi = (int)xlane<2>((uint32_t)bi); break;
        }
        best_merge(bv, bi, ov, oi);
      }
      bi = __builtin_amdgcn_readfirstlane(bi);
      // a timed-out poll leaves the error word set and may leave garbage: keep the id in range
      return (bi >= 0 && bi < (a.cp_frame ? a.cp_vocab : a.vocab)) ? bi : 0;
    }
    const int n = a.cp_frame ? a.cp_vocab : a.vocab;
    poll_vec_long(P, ws->logits[pi & 1], n, a.tag_base + TAG_HEAD + (uint32_t)pi, s.stage);
    SelParams sp = a.sel;
    sp.seed = SIO(seed);
    if (a.cp_frame) {
      sp.group = pi;   // CP head pi-1 selects codebook group pi
    } else {
      // suppress ids [V-1024, V) except EOS (generator.py:71-75)
      if (a.mask_tail)
        for (int i = lane; i < n; i += 64)
          if (i >= n - 1024 && i != a.eos_id) s.stage[i] = -INFINITY;
      // repetition penalty, once per distinct id (generator.py:161-167)
      if (a.rep_penalty != 1.0f && SIO(n_history) > 0) {
        for (int i = lane; i < MAXV / 32; i += 64) s.pen_bits[i] = 0u;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        for (int i = lane; i < SIO(n_history); i += 64) {
          const int id = SIO(history[i]);
          if (id >= 0 && id < n) atomicOr(&s.pen_bits[id >> 5], 1u << (id & 31));
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        for (int i = lane; i < n; i += 64) {
          if (s.pen_bits[i >> 5] & (1u << (i & 31))) {
            const float v = s.stage[i];   // bf16 arithmetic of the reference: the result is rounded to bf16
            s.stage[i] = rbf(v > 0.f ? v / a.rep_penalty : v * a.rep_penalty);
          }
        }
      }
      if (a.suppress_eos && a.eos_id >= 0 && a.eos_id < n && lane == 0) s.stage[a.eos_id] = -INFINITY;
      sp.group = 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return wave_select(s.stage, n, sp, &s.sel);
  };

  // =====================================================================================
  // Step schedule. One walker defines the barrier sequence; the poller wave and the math
  // waves each run it with their own action, in separate loops (so the math waves' weight
  // tiles and the poller's poll registers are never live at the same time). Math waves run
  // the compute of step k on operands the poller prepared during step k-1 and then issue the
  // weight tile of step k+1.
  // =====================================================================================
  enum Step { S_PRO, S_QKV, S_ATT, S_O, S_GU, S_DOWN, S_HEAD, S_QKV2, S_ATT2, S_GU2, S_DOWN2 };
  int nstep = 0;
  auto stamp = [&]() {
    if (a.trace != nullptr && lane == 0 && (poller || mw == 0) && nstep < TRACE_STEPS)
      a.trace[((size_t)wg * TRACE_STEPS + nstep) * 2 + (poller ? 1 : 0)] = __builtin_amdgcn_s_memrealtime();
    ++nstep;
  };
  // attention over the whole context in every workgroup when it fits one pass of the math
  // waves (attention and O projection then share a step); split into chunks otherwise
  auto att_local = [&](int pi) { return SIO(pos0) + pi + 1 <= KVGeo<BB>::SUB; };
  // the code-predictor frame's position 0 feeds no head: of its last layer only the K/V entry
  // (the QKV step) is read later, so its attention, MLP and final norm are not computed
  auto kv_only = [&](int pi, int layer) { return a.cp_frame && pi == 0 && layer == NL - 1 && a.n_pos > 1; };
  // The code-predictor frame (batch 1) runs positions 0 and 1 as one two-column pass: both
  // inputs are known at launch (bf16(h) and emb_bb[g0]), position 1's layer l attends to
  // position 0's layer-l entry, and every weight tile serves both columns. Its steps: the
  // *2 variants, indexed by position 1; a head follows, then positions 2.. one by one.
  const bool duo_frame = DUO_OK && a.cp_frame && a.n_pos >= 2;
  auto walk = [&](auto&& act) {
    act(S_PRO, 0, 0); stamp();
    step_barrier();
    int pi_first = 0;
    if (duo_frame) {
      for (int layer = 0; layer < NL; ++layer) {
        act(S_QKV2, 1, layer); stamp(); step_barrier();
        act(S_ATT2, 1, layer); stamp(); step_barrier();
        act(S_GU2, 1, layer); stamp(); step_barrier();
        act(S_DOWN2, 1, layer); stamp(); step_barrier();
      }
      act(S_HEAD, 1, NL - 1); stamp(); step_barrier();
      pi_first = 2;
    }
    for (int pi = pi_first; pi < a.n_pos; ++pi) {
      for (int layer = 0; layer < NL; ++layer) {
        act(S_QKV, pi, layer); stamp(); step_barrier();
        if (kv_only(pi, layer)) continue;
        act(S_ATT, pi, layer); stamp(); step_barrier();
        if (!att_local(pi)) { act(S_O, pi, layer); stamp(); step_barrier(); }
        act(S_GU, pi, layer); stamp(); step_barrier();
        act(S_DOWN, pi, layer); stamp(); step_barrier();
      }
      if (has_head(pi)) { act(S_HEAD, pi, NL - 1); stamp(); step_barrier(); }
    }
  };
  struct PosInfo { int pos, L, C, P, c0, c1; bool local, has_chunk, last_pos, head; };
  auto pinfo = [&](int pi) {
    PosInfo q;
    q.pos = SIO(pos0) + pi;
    q.L = q.pos + 1;
    chunking<BB>(q.L, q.C, q.P);
    q.local = att_local(pi);
    // chunked: unit u = (chunk u >> 1, query head u & 1) of the XCD's KV head; workgroup li takes
    // unit li (XL: units lu, lu + 4, lu + 8, lu + 12 with lu = li_hw >> 3; these fields are lu's)
    const int lu = XL ? (li_hw >> 3) : li;
    q.has_chunk = q.local || lu < 2 * q.C;
    q.c0 = q.local ? 0 : (lu >> 1) * q.P;
    q.c1 = q.local ? q.L : min(q.L, ((lu >> 1) + 1) * q.P);
    q.last_pos = pi == a.n_pos - 1;
    q.head = has_head(pi);
    return q;
  };
  // Tiles are (re)defined on every path so that no stale tile value stays live across the
  // step loop (that would keep all tiles resident at once and spill).

  if (poller) {
    int npass = 0;   // layer passes begun
    walk([&](int st, int pi, int layer) {
      lane = opaque(lane);
      if (st == S_QKV || st == S_QKV2) {
        if (npass > 0) P.ec.spin_cap = a.spin_cap;
        ++npass;
      }
      const PosInfo q = pinfo(pi);
      const int lp = pi * NL + layer;
      const int nl = layer + 1 < NL ? layer + 1 : 0;   // next layer pass (wraps to the next position)
      switch (st) {
        case S_PRO:
          if (a.cp_frame) {
            if (lane < a.n_groups) s.embp[lane] = a.cp_embs[lane];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          }
          if (pen_rows) {
            // ids in the history, once per distinct id (generator.py:161-167); read by the head rows
            for (int i = lane; i < MAXV / 32; i += 64) s.pen_bits[i] = 0u;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            for (int i = lane; i < SIO(n_history); i += 64) {
              const int id = SIO(history[i]);
              if (id >= 0 && id < a.vocab) atomicOr(&s.pen_bits[id >> 5], 1u << (id & 31));
            }
          }
          load_gain_pairs(g_in, lw(LW, 0, W_LNIN));
          load_gain_pairs(g_post, lw(LW, 0, W_LNPOST));
          load_gain_pairs(g_fin, a.final_norm);
          load_qk_gains(0);
          load_rope(q.pos);
          prep_input0(0, Col0{});
          if constexpr (DUO_OK) {
            if (duo_frame) {
              prep_input0(1, Col1{});
              if (lead) comb_add(true, Col1{});   // emb_bb[g0] opens the combine
              load_rope_to(q.pos + 1, rc1, rsn1);
            }
          }
          load_gain_pairs(g_in, lw(LW, NL > 1 ? 1 : 0, W_LNIN));
          break;
        case S_QKV: {
          const bool rope_next = layer == NL - 1 && !q.last_pos;
          load_qk_gains_to(nl, qn_n, kn_n);
          if (rope_next) load_rope_to(q.pos + 1, rc_n, rsn_n);
          prep_att(lp, layer, q.pos, q.C, Col0{});
          take2(qn, qn_n);
          take2(kn, kn_n);
          if (rope_next) { take2(rc, rc_n); take2(rsn, rsn_n); }
          if (kv_only(pi, layer)) {
            // position 1's input, in place of this position's DOWN step; the math waves read
            // xn before publishing the QKV rows prep_att has waited for, so xn is free
            prep_input0(pi + 1, Col0{});
            if (lead) comb_add(true, Col0{});
            load_gain_pairs(g_in, lw(LW, NL > 1 ? 1 : 0, W_LNIN));
            load_gain_pairs(g_post, lw(LW, 0, W_LNPOST));
          }
          break;
        }
        case S_ATT:
          // the math waves' attention synchronises the whole workgroup (passes + 2 times);
          // this wave's inputs for the step are produced after those points anyway
          if (q.has_chunk) {
            int nb = (q.c1 - q.c0 + KVGeo<BB>::SUB - 1) / KVGeo<BB>::SUB + 2;
            if (XL && !q.local) {
              // the workgroup's further units
              for (int u = (li_hw >> 3) + 4; u < 2 * q.C; u += 4) {
                const int c0 = (u >> 1) * q.P, c1 = min(q.L, c0 + q.P);
                nb += (c1 - c0 + KVGeo<BB>::SUB - 1) / KVGeo<BB>::SUB + 2;
              }
            }
            for (int b = 0; b < nb; ++b) step_barrier();
          }
          if (q.local) {
            load_gain_pairs(g_post_n, lw(LW, nl, W_LNPOST));
            prep_gu(lp, layer, Col0{});
            take8(g_post, g_post_n);
          } else {
            prep_o(lp, q.C);
          }
          break;
        case S_O:
          load_gain_pairs(g_post_n, lw(LW, nl, W_LNPOST));
          prep_gu(lp, layer, Col0{});
          take8(g_post, g_post_n);
          break;
        case S_GU: prep_down(lp, Col0{}); break;
        case S_DOWN: {
          // g_in then serves the layer after next
          const bool gin_next = layer < NL - 1 || !(q.head || q.last_pos);
          if (gin_next) load_gain_pairs(g_in_n, lw(LW, (nl + 1) % NL, W_LNIN));
          if (layer < NL - 1) { ar2(lp, Col0{}); prep_input_next(lp, Col0{}); }
          else if (q.head || q.last_pos) { ar2(lp, Col0{}); prep_final(lp, Col0{}); }
          else {
            prep_input0(pi + 1, Col0{});
            if (a.cp_frame && lead) comb_add(pi == 0, Col0{});
          }
          if (gin_next) take8(g_in, g_in_n);
          break;
        }
        case S_QKV2:
          if constexpr (DUO_OK) {
            load_qk_gains_to(nl, qn_n, kn_n);
            if (layer == NL - 1) load_rope_to(q.pos + 1, rc_n, rsn_n);
            prep_att(lp - NL, layer, q.pos - 1, q.C, Col0{});
            prep_att(lp, layer, q.pos, q.C, Col1{});
            take2(qn, qn_n);
            take2(kn, kn_n);
            if (layer == NL - 1) { take2(rc, rc_n); take2(rsn, rsn_n); }
          }
          break;
        case S_ATT2:
          if constexpr (DUO_OK) {
            load_gain_pairs(g_post_n, lw(LW, nl, W_LNPOST));
            for (int b = 0; b < 3; ++b) step_barrier();   // the local attention's three barriers
            // position 0's last layer feeds nothing beyond its K/V entry; both columns' sums are
            // published before either gather, so neither gather waits behind the other's
            if (layer < NL - 1) ar1(lp - NL, Col0{});
            ar1(lp, Col1{});
            if (layer < NL - 1) gather_h1(lp - NL, Col0{});
            gather_h1(lp, Col1{});
            take8(g_post, g_post_n);
          }
          break;
        case S_GU2:
          if constexpr (DUO_OK) {
            if (layer < NL - 1) prep_down(lp - NL, Col0{});
            prep_down(lp, Col1{});
          }
          break;
        case S_DOWN2:
          if constexpr (DUO_OK) {
            if (layer < NL - 1) {
              load_gain_pairs(g_in_n, lw(LW, (nl + 1) % NL, W_LNIN));
              ar2(lp - NL, Col0{});
              ar2(lp, Col1{});
              prep_input_next(lp - NL, Col0{});
              prep_input_next(lp, Col1{});
              take8(g_in, g_in_n);
            } else {
              ar2(lp, Col1{});
              prep_final(lp, Col1{});
            }
          }
          break;
        case S_HEAD:
          if (a.cp_frame && !q.last_pos) load_gain_pairs(g_in_n, lw(LW, NL > 1 ? 1 : 0, W_LNIN));
          // greedy backbone head: workgroup 0 of every XCD takes part in the candidate exchange
          if (a.cp_frame || lead || (greedy_sel && !XL && li == 0)) {
            const int tok = select(pi);
            if (a.cp_frame) {
              if (lane == 0) s.tok[pi - 1] = tok;
              __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
              if (!q.last_pos) {
                prep_input0(pi + 1, Col0{});
                if (lead) comb_add(false, Col0{});
                take8(g_in, g_in_n);
              }
            } else if (lead && lane == 0 && SIO(out_token)) {
              *SIO(out_token) = tok;
            }
          }
          break;
      }
    });
  } else {
    walk([&](int st, int pi, int layer) {
      lane = opaque(lane);
      const PosInfo q = pinfo(pi);
      const int lp = pi * NL + layer;
      const bool last_layer = layer == NL - 1;
      // Each tile is loaded one step ahead of its use, right after the step's own compute,
      // so at most the tile in use and the next one are live.
      // XL: a GEMV stage runs the workgroup's 8 row groups; each group's tile is issued one group
      // ahead into the second register set (the first group's a step ahead, as in batch 1). The
      // last pair is peeled off the loop so that no tile load sits under a branch: the compiler
      // then waits only for the tile in use, not for the one in flight behind it.
      auto qkv_stage = [&](int layer_) {
        if constexpr (XL) {
          TileQKV t1;
#pragma unroll 1
          for (int sub = 0; sub < NSUB - 2; sub += 2) {
            load_qkv<BB>(t1, LW, layer_, xcd, li + sub + 1, mw, lane);
            math_qkv(lp, li + sub, tq, Col0{});
            load_qkv<BB>(tq, LW, layer_, xcd, li + sub + 2, mw, lane);
            math_qkv(lp, li + sub + 1, t1, Col0{});
          }
          load_qkv<BB>(t1, LW, layer_, xcd, li + NSUB - 1, mw, lane);
          math_qkv(lp, li + NSUB - 2, tq, Col0{});
          math_qkv(lp, li + NSUB - 1, t1, Col0{});
        } else {
          math_qkv(lp, li, tq, Col0{});
        }
      };
      auto o_stage = [&](int layer_) {
        if constexpr (XL) {
          TileO t1;
#pragma unroll 1
          for (int sub = 0; sub < NSUB - 2; sub += 2) {
            load_o<BB>(t1, LW, layer_, xcd, li + sub + 1, mw, lane);
            math_o(lp, li + sub, to, Col0{});
            load_o<BB>(to, LW, layer_, xcd, li + sub + 2, mw, lane);
            math_o(lp, li + sub + 1, t1, Col0{});
          }
          load_o<BB>(t1, LW, layer_, xcd, li + NSUB - 1, mw, lane);
          math_o(lp, li + NSUB - 2, to, Col0{});
          math_o(lp, li + NSUB - 1, t1, Col0{});
        } else {
          math_o(lp, li, to, Col0{});
        }
      };
      auto gu_stage = [&](int layer_) {
        if constexpr (XL) {
          TileGU t1;
#pragma unroll 1
          for (int sub = 0; sub < NSUB - 2; sub += 2) {
            load_gu<BB>(t1, LW, layer_, xcd, li + sub + 1, mw, lane);
            math_gu(lp, li + sub, tgu, Col0{});
            load_gu<BB>(tgu, LW, layer_, xcd, li + sub + 2, mw, lane);
            math_gu(lp, li + sub + 1, t1, Col0{});
          }
          load_gu<BB>(t1, LW, layer_, xcd, li + NSUB - 1, mw, lane);
          math_gu(lp, li + NSUB - 2, tgu, Col0{});
          math_gu(lp, li + NSUB - 1, t1, Col0{});
        } else {
          math_gu(lp, li, tgu, Col0{});
        }
      };
      auto down_stage = [&](int layer_) {
        if constexpr (XL) {
          TileD t1;
#pragma unroll 1
          for (int sub = 0; sub < NSUB - 2; sub += 2) {
            load_d<BB>(t1, LW, layer_, xcd, li + sub + 1, mw, lane);
            math_down(lp, li + sub, td, Col0{});
            load_d<BB>(td, LW, layer_, xcd, li + sub + 2, mw, lane);
            math_down(lp, li + sub + 1, t1, Col0{});
          }
          load_d<BB>(t1, LW, layer_, xcd, li + NSUB - 1, mw, lane);
          math_down(lp, li + NSUB - 2, td, Col0{});
          math_down(lp, li + NSUB - 1, t1, Col0{});
        } else {
          math_down(lp, li, td, Col0{});
        }
      };
      auto head_stage = [&]() {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        if constexpr (XL) {
          TileQKV t1;
          int row0, nrows;
#pragma unroll 1
          for (int sub = 0; sub < NSUB - 2; sub += 2) {
            head_rows(sub + 1, row0, nrows);
            load_head<BB>(t1, head_weights(pi), row0, nrows, lane);
            head_group(pi, sub, tq, bv, bi);
            head_rows(sub + 2, row0, nrows);
            load_head<BB>(tq, head_weights(pi), row0, nrows, lane);
            head_group(pi, sub + 1, t1, bv, bi);
          }
          head_rows(NSUB - 1, row0, nrows);
          load_head<BB>(t1, head_weights(pi), row0, nrows, lane);
          head_group(pi, NSUB - 2, tq, bv, bi);
          head_group(pi, NSUB - 1, t1, bv, bi);
        } else {
          head_group(pi, 0, tq, bv, bi);
        }
        head_publish(pi, bv, bi);
      };
      switch (st) {
        case S_PRO:
          load_qkv<BB>(tq, LW, 0, xcd, li, mw, lane);
          break;
        case S_QKV:
          qkv_stage(layer);
          if (kv_only(pi, layer)) {
            // the next step is position 1's layer-0 QKV
            tk = TileKV<BB>{};
            load_qkv<BB>(tq, LW, 0, xcd, li, mw, lane);
            break;
          }
          if (q.has_chunk) load_kv<BB>(tk, a, SIO(kc), SIO(vc), layer, xcd, q.c0, min(q.c1, q.L - 1), mw, lane);
          else tk = TileKV<BB>{};
          if (q.local) load_o<BB>(to, LW, layer, xcd, li, mw, lane);
          break;
        case S_ATT:
          if constexpr (!BB) {
            if (q.local) attention_cp_local(q.L, std::false_type{});
            else if (q.has_chunk) attention(std::integral_constant<int, 1>{}, lp, layer, q.L, q.c0, q.c1, false, li & 1, li);
          } else if (q.has_chunk) {
            if (q.local) {
              attention(std::integral_constant<int, 2>{}, lp, layer, q.L, q.c0, q.c1, true, 0, li);
            } else if constexpr (XL) {
              // units lu, lu + 4, ... (the first one's KV tile was issued in the QKV step)
              for (int u = li_hw >> 3; u < 2 * q.C; u += 4) {
                const int c0 = (u >> 1) * q.P, c1 = min(q.L, c0 + q.P);
                if (u >= 4) load_kv<BB>(tk, a, SIO(kc), SIO(vc), layer, xcd, c0, min(c1, q.L - 1), mw, lane);
                attention(std::integral_constant<int, 1>{}, lp, layer, q.L, c0, c1, false, u & 1, u);
              }
            } else {
              attention(std::integral_constant<int, 1>{}, lp, layer, q.L, q.c0, q.c1, false, li & 1, li);
            }
          }
          if (q.local) {
            o_stage(layer);
            load_gu_paced<BB>(tgu, LW, layer, xcd, li, mw, lane);
          } else {
            load_o<BB>(to, LW, layer, xcd, li, mw, lane);
          }
          break;
        case S_O:
          o_stage(layer);
          load_gu_paced<BB>(tgu, LW, layer, xcd, li, mw, lane);
          break;
        case S_GU:
          gu_stage(layer);
          load_d<BB, 12>(td, LW, layer, xcd, li, mw, lane);
          break;
        case S_DOWN:
          down_stage(layer);
          if (!last_layer) {
            if constexpr (BB) load_qkv<BB>(tq, LW, layer + 1, xcd, li, mw, lane);
            else load_qkv<BB, 16>(tq, LW, layer + 1, xcd, li, mw, lane);
          } else if (q.head) {
            int row0, nrows;
            head_rows(0, row0, nrows);
            load_head<BB, 16>(tq, head_weights(pi), row0, nrows, lane);
          } else if (!q.last_pos) {
            load_qkv<BB>(tq, LW, 0, xcd, li, mw, lane);
          } else {
            tq = TileQKV{};
          }
          break;
        case S_HEAD:
          head_stage();
          if (!q.last_pos) load_qkv<BB, 16>(tq, LW, 0, xcd, li, mw, lane);
          else tq = TileQKV{};
          break;
        case S_QKV2:
          if constexpr (DUO_OK) {
            math_qkv(lp - NL, li, tq, Col0{});
            math_qkv(lp, li, tq, Col1{});
            tk = TileKV<BB>{};
            load_o<BB>(to, LW, layer, xcd, li, mw, lane);
          }
          break;
        case S_ATT2:
          if constexpr (DUO_OK) {
            attention_cp_local(2, std::true_type{});
            math_o(lp - NL, li, to, Col0{});
            math_o(lp, li, to, Col1{});
            load_gu_paced<BB>(tgu, LW, layer, xcd, li, mw, lane);
          }
          break;
        case S_GU2:
          if constexpr (DUO_OK) {
            math_gu(lp - NL, li, tgu, Col0{});
            math_gu(lp, li, tgu, Col1{});
            load_d<BB>(td, LW, layer, xcd, li, mw, lane);
          }
          break;
        case S_DOWN2:
          if constexpr (DUO_OK) {
            math_down(lp - NL, li, td, Col0{});
            math_down(lp, li, td, Col1{});
            if (!last_layer) {
              load_qkv<BB, 16>(tq, LW, layer + 1, xcd, li, mw, lane);
            } else {
              int row0, nrows;
              head_rows(0, row0, nrows);
              load_head<BB, 16>(tq, head_weights(pi), row0, nrows, lane);
            }
          }
          break;
      }
    });
  }

  // ---- code-predictor frame epilogue: tokens and the bf16 embedding combine
  if (a.cp_frame && lead && poller) {
    if (lane == 0) {
      if (SIO(hist_slot)) *SIO(hist_slot) = g0;
      SIO(out_tokens[0]) = g0;
      for (int g = 0; g < a.n_groups; ++g) SIO(out_tokens[1 + g]) = s.tok[g];
    }
    // s.comb holds emb_bb[g0] + emb_0[t_0] + ... + emb_{n-2}[t_{n-2}] (each row was loaded as a
    // position's input); the last group's row and the text row complete it (generator.py:356-362)
    const int gl = a.n_groups - 1;
    const auto* lr = gmem(reinterpret_cast<const uint32_t*>(s.embp[gl] + (size_t)s.tok[gl] * HID));
    uint32_t wl[8], wt[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) wl[k] = lr[lane + 64 * k];
    if (SIO(text_row)) {
      const auto* tr = gmem(reinterpret_cast<const uint32_t*>(SIO(text_row)));
#pragma unroll
      for (int k = 0; k < 8; ++k) wt[k] = tr[lane + 64 * k];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = 2 * (lane + 64 * k);
      float a0 = rbf(s.comb[e] + bflo(wl[k])), a1 = rbf(s.comb[e + 1] + bfhi(wl[k]));
      if (SIO(text_row)) { a0 = rbf(a0 + bflo(wt[k])); a1 = rbf(a1 + bfhi(wt[k])); }
      gput(reinterpret_cast<uint32_t*>(SIO(out_combined)) + (e >> 1), (uint32_t)f2bf(a0) | ((uint32_t)f2bf(a1) << 16));
    }
  }
}

#undef SIO

template __global__ void qtts_decode_kernel<true, false>(const KArgs a);
template __global__ void qtts_decode_kernel<false, false>(const KArgs a);
template __global__ void qtts_decode_kernel<false, true>(const KArgs a);
template __global__ void qtts_decode_kernel<true, true>(const KArgs a);

}  // namespace qtts

// =========================================================================================
// Host side
// =========================================================================================
namespace {

using qtts::KArgs;
using qtts::Workspace;

using qtts_host::kSpinCap;
constexpr uint32_t kSeqLimit = (1u << 20) - 1u;  // tag = (sequence << 12) | (layer pass * 8 + slot)

struct DeviceCheck {
  bool done = false;
  hipError_t status = hipSuccess;
  // Ordering of this library's launches on the device: a launch on another stream than the
  // previous one first waits for it. Two persistent launches that overlapped could each hold
  // part of the CUs while waiting for workgroups of their own that cannot be placed.
  hipEvent_t last = nullptr;
  hipStream_t last_stream = nullptr;
  bool has_last = false;
  void* scratch = nullptr;   // device address of this device's copy of `scratch`
};
std::mutex g_mu;
std::unordered_map<int, DeviceCheck> g_dev;
// Launch sequence of every workspace, keyed by its device address: the tag base of the next
// launch that uses it. Absent = never used (or released): its first launch zero-fills it.
std::unordered_map<const void*, uint32_t> g_seq;
// Library-owned workspaces of the reference-compatible launchers, one per (device, stream):
// launches on one stream are ordered, so they never overlap on a workspace.
std::map<std::pair<int, hipStream_t>, void*> g_lib_ws;
uint64_t* g_trace = nullptr;   // optional step timeline buffer
// cap of the first layer pass's waits in every persistent launch (qtts_debug_entry_spin_cap)
std::atomic<uint32_t> g_entry_cap{qtts_host::kEntrySpinCap};

// XCC id of every workgroup of the probe launch (a static device array: the set-up allocates nothing)
__device__ int g_xcc_probe[qtts::NWG];

// Exchange workspace of launch_tts_decode_with_embedding_static: one Workspace per device,
// held until the process ends. In host code `scratch` is only a handle for
// hipGetSymbolAddress; the device address is kept per device in DeviceCheck::scratch.
constexpr size_t kStaticScratchBytes = sizeof(Workspace);
static_assert(kStaticScratchBytes == QTTS_STATIC_SCRATCH_BYTES, "QTTS_STATIC_SCRATCH_BYTES must equal sizeof(Workspace)");
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

__global__ void xcc_probe_kernel() {
  if (threadIdx.x == 0) g_xcc_probe[blockIdx.x] = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u);
}
__global__ void zero_kernel(uint4* p, size_t n16) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

// gfx950 with 256 CUs, room for one workgroup of every instantiation on each CU (so a launch of
// 256 workgroups is co-resident when the device is not shared with other kernels), and workgroup
// b placed on XCC (b + r) % 8 for a fixed rotation r, 32 workgroups per XCD. Every in-kernel wait
// is bounded, so a launch that is not co-resident ends with the error word set instead of hanging.
// Runs its HIP calls with `device` current (the caller's current device is restored).
hipError_t check_device_locked(int device, DeviceCheck& dc);
hipError_t check_device(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceCheck& dc = g_dev[device];
  if (dc.done) return dc.status;
  dc.done = true;
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return dc.status = e;
  if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return dc.status = e;
  dc.status = check_device_locked(device, dc);
  if (cur != device && (e = hipSetDevice(cur)) != hipSuccess && dc.status == hipSuccess) dc.status = e;
  return dc.status;
}
hipError_t check_device_locked(int device, DeviceCheck& dc) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return e;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0 || prop.multiProcessorCount != qtts::NWG)
    return hipErrorInvalidDevice;
  const void* fns[] = {(const void*)qtts::qtts_decode_kernel<true, false>, (const void*)qtts::qtts_decode_kernel<false, false>,
                       (const void*)qtts::qtts_decode_kernel<false, true>, (const void*)qtts::qtts_decode_kernel<true, true>};
  for (const void* fn : fns) {
    int occ = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, qtts::NTHR, 0);
    if (e != hipSuccess || occ < 1) return e != hipSuccess ? e : hipErrorInvalidDevice;
  }
  hipLaunchKernelGGL(xcc_probe_kernel, dim3(qtts::NWG), dim3(64), 0, 0);
  e = hipGetLastError();
  int h[qtts::NWG];
  if (e == hipSuccess) e = hipMemcpyFromSymbol(h, HIP_SYMBOL(g_xcc_probe), sizeof(h), 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return e;
  int count[16] = {0};
  for (int b = 0; b < qtts::NWG; ++b) {
    if (h[b] < 0 || h[b] >= qtts::NXCD || ((h[b] - b) & 7) != ((h[0] - 0) & 7)) return hipErrorInvalidDevice;
    ++count[h[b]];
  }
  for (int x = 0; x < qtts::NXCD; ++x)
    if (count[x] != qtts::WPX) return hipErrorInvalidDevice;
  if ((e = hipEventCreateWithFlags(&dc.last, hipEventDisableTiming)) != hipSuccess) return e;
  // this device's copy of the static exchange workspace (the no-allocation entry point's)
  if ((e = hipGetSymbolAddress(&dc.scratch, HIP_SYMBOL(scratch))) != hipSuccess) return e;
  if (dc.scratch == nullptr || (reinterpret_cast<uintptr_t>(dc.scratch) & 255u) != 0) return hipErrorInvalidSymbol;
  return hipSuccess;
}

// Tag base of a launch over the n consecutive workspaces of `bytes` each at ws. The launch takes
// the largest sequence of its workspaces and moves all n past it, so its tags differ from every
// tag they hold. When one of them is new, or the sequence space is used up, exactly these n
// workspaces are zero-filled (a fill kernel on the launch stream) and the sequence restarts at 1.
// Called with g_mu held.
uint32_t next_tag_base(void* ws, int n, size_t bytes, hipStream_t stream, hipError_t* err) {
  uint32_t seq = 0;
  bool fresh = false;
  for (int i = 0; i < n; ++i) {
    const auto it = g_seq.find(reinterpret_cast<char*>(ws) + (size_t)i * bytes);
    if (it == g_seq.end()) fresh = true;
    else seq = it->second > seq ? it->second : seq;
  }
  *err = hipSuccess;
  if (fresh || seq == 0 || seq >= kSeqLimit) {
    hipLaunchKernelGGL(zero_kernel, dim3(256), dim3(256), 0, stream, reinterpret_cast<uint4*>(ws),
                       (size_t)n * bytes / 16);
    *err = hipGetLastError();
    seq = 1;
  }
  for (int i = 0; i < n; ++i) g_seq[reinterpret_cast<char*>(ws) + (size_t)i * bytes] = seq + 1;
  return seq << 12;
}

// Ordered launch of a persistent kernel: a launch on another stream than the library's previous
// one on this device first waits for it. Called with the device checked.
hipError_t ordered_launch(int dev, const void* fn, int threads, void* kargs, uint32_t* tag_base, void* ws, int n_ws,
                          size_t ws_bytes, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceCheck& dc = g_dev[dev];
  hipError_t e = hipSuccess;
  if (dc.has_last && dc.last_stream != stream && (e = hipStreamWaitEvent(stream, dc.last, 0)) != hipSuccess) return e;
  hipError_t ze = hipSuccess;
  *tag_base = next_tag_base(ws, n_ws, ws_bytes, stream, &ze);
  if (ze != hipSuccess) return ze;
  void* args[] = {kargs};
  if ((e = hipLaunchKernel(fn, dim3(qtts::NWG), dim3(threads), args, 0, stream)) != hipSuccess) return e;
  if ((e = hipEventRecord(dc.last, stream)) != hipSuccess) return e;
  dc.last_stream = stream;
  dc.has_last = true;
  return hipSuccess;
}

// xl: one stream per XCD, n_streams workspaces of one block starting at a.io[0].ws
hipError_t launch(bool bb, KArgs& a, hipStream_t stream, bool xl = false, int n_streams = 1) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if ((e = check_device(dev)) != hipSuccess) return e;
  if (a.num_layers < 1 || a.n_pos < 1 || a.num_layers * a.n_pos > qtts::MAX_LAYER_PASSES) return hipErrorInvalidValue;
  if (a.io[0].pos0 < 0 || a.io[0].pos0 + a.n_pos > a.max_seq) return hipErrorInvalidValue;
  a.spin_cap = kSpinCap;
  a.entry_spin_cap = g_entry_cap.load(std::memory_order_relaxed);
  a.trace = g_trace;
  const void* fn = bb ? (xl ? (const void*)qtts::qtts_decode_kernel<true, true> : (const void*)qtts::qtts_decode_kernel<true, false>)
                      : (xl ? (const void*)qtts::qtts_decode_kernel<false, true> : (const void*)qtts::qtts_decode_kernel<false, false>);
  return ordered_launch(dev, fn, qtts::NTHR, &a, &a.tag_base, a.io[0].ws, n_streams, sizeof(Workspace), stream);
}

void* lib_workspace(hipStream_t stream, hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  void*& p = g_lib_ws[{dev, stream}];
  if (p == nullptr) {
    *err = hipMalloc(&p, sizeof(Workspace));
    if (*err != hipSuccess) { p = nullptr; return nullptr; }
    g_seq.erase(p);   // a new workspace: its first launch zero-fills it
  }
  return p;
}

void base_args(KArgs& a, const TTSLayerWeights* layers, int num_layers, const void* final_norm, const void* cos_t,
               const void* sin_t, void* kc, void* vc, int max_seq) {
  std::memset(&a, 0, sizeof(a));
  a.layers = layers;
  a.num_layers = num_layers;
  a.final_norm = reinterpret_cast<const qtts::bf16_t*>(final_norm);
  a.cos_t = reinterpret_cast<const qtts::bf16_t*>(cos_t);
  a.sin_t = reinterpret_cast<const qtts::bf16_t*>(sin_t);
  a.io[0].kc = kc;
  a.io[0].vc = vc;
  a.max_seq = max_seq;
  a.scale = 0.08838834764831845f;
  a.eos_id = -1;
  a.n_pos = 1;
  a.sel.temperature = 1.0f;
  a.sel.top_p = 1.0f;
}

// static_ws: use this device's static exchange workspace instead of the library-owned one
hipError_t ref_launch(bool bb, int token, const void* embed, const void* emb, const TTSLayerWeights* layers,
                      const void* final_norm, const void* cos_t, const void* sin_t, void* kc, void* vc,
                      void* hidden_buffer, void* g_normalized, int num_layers, int position, int cache_len,
                      int max_seq_len, float attn_scale, hipStream_t stream, bool static_ws = false) {
  if (cache_len != position + 1 || position < 0 || position >= max_seq_len) return hipErrorInvalidValue;
  if (layers == nullptr || final_norm == nullptr || cos_t == nullptr || sin_t == nullptr || kc == nullptr || vc == nullptr ||
      g_normalized == nullptr || (emb == nullptr && embed == nullptr))
    return hipErrorInvalidValue;
  hipError_t e;
  void* ws = nullptr;
  if (static_ws) {
    int dev = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = check_device(dev)) != hipSuccess) return e;   // first call on a device: set-up, scratch address
    std::lock_guard<std::mutex> lk(g_mu);
    ws = g_dev[dev].scratch;
    if (ws == nullptr) return hipErrorInvalidSymbol;
  } else {
    ws = lib_workspace(stream, &e);
    if (ws == nullptr) return e;
  }
  KArgs a;
  base_args(a, layers, num_layers, final_norm, cos_t, sin_t, kc, vc, max_seq_len);
  a.scale = attn_scale;
  a.io[0].ws = reinterpret_cast<Workspace*>(ws);
  a.io[0].pos0 = position;
  a.io[0].pos3[0] = a.io[0].pos3[1] = a.io[0].pos3[2] = position;
  a.io[0].in_emb = reinterpret_cast<const qtts::bf16_t*>(emb);
  a.embed_w = reinterpret_cast<const qtts::bf16_t*>(embed);
  a.io[0].in_tok = token;
  a.io[0].out_hidden = reinterpret_cast<float*>(g_normalized);
  a.io[0].out_residual = hidden_buffer;
  return launch(bb, a, stream);
}

}  // namespace

namespace qtts_host {

hipError_t check_kernel(const void* fn, int threads, int* device) {
  hipError_t e = hipGetDevice(device);
  if (e != hipSuccess) return e;
  if ((e = check_device(*device)) != hipSuccess) return e;
  static std::map<std::pair<int, const void*>, hipError_t> checked;   // guarded by g_mu
  std::lock_guard<std::mutex> lk(g_mu);
  const auto key = std::make_pair(*device, fn);
  const auto it = checked.find(key);
  if (it != checked.end()) return it->second;
  int occ = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, threads, 0);
  if (e == hipSuccess && occ < 1) e = hipErrorInvalidDevice;
  checked[key] = e;
  return e;
}

hipError_t launch_persistent(const void* fn, int threads, void* kargs, uint32_t* tag_base, void* ws, int n_ws,
                             size_t ws_bytes, hipStream_t stream) {
  int dev = 0;
  hipError_t e = check_kernel(fn, threads, &dev);
  if (e != hipSuccess) return e;
  return ordered_launch(dev, fn, threads, kargs, tag_base, ws, n_ws, ws_bytes, stream);
}

uint32_t entry_spin_cap() { return g_entry_cap.load(std::memory_order_relaxed); }

}  // namespace qtts_host

extern "C" {

hipError_t launch_tts_decode(int input_token_id, const void* embed_weight, const TTSLayerWeights* layer_weights,
                             const void* final_norm_weight, const void* cos_table, const void* sin_table, void* k_cache,
                             void* v_cache, void* hidden_buffer, void*, void*, void*, void*, void*, void*, void*,
                             void* g_normalized, int num_layers, int position, int cache_len, int max_seq_len,
                             float attn_scale, hipStream_t stream) {
  if (embed_weight == nullptr || input_token_id < 0) return hipErrorInvalidValue;
  return ref_launch(true, input_token_id, embed_weight, nullptr, layer_weights, final_norm_weight, cos_table, sin_table,
                    k_cache, v_cache, hidden_buffer, g_normalized, num_layers, position, cache_len, max_seq_len,
                    attn_scale, stream);
}

hipError_t launch_tts_decode_with_embedding(const void* input_embedding, const TTSLayerWeights* layer_weights,
                                            const void* final_norm_weight, const void* cos_table, const void* sin_table,
                                            void* k_cache, void* v_cache, void* hidden_buffer, void*, void*, void*,
                                            void*, void*, void*, void*, void* g_normalized, int num_layers,
                                            int position, int cache_len, int max_seq_len, float attn_scale,
                                            hipStream_t stream) {
  if (input_embedding == nullptr) return hipErrorInvalidValue;
  return ref_launch(true, 0, nullptr, input_embedding, layer_weights, final_norm_weight, cos_table, sin_table, k_cache,
                    v_cache, hidden_buffer, g_normalized, num_layers, position, cache_len, max_seq_len, attn_scale,
                    stream);
}

hipError_t launch_tts_decode_with_embedding_static(const void* input_embedding, const TTSLayerWeights* layer_weights,
                                                   const void* final_norm_weight, const void* cos_table,
                                                   const void* sin_table, void* k_cache, void* v_cache,
                                                   void* hidden_buffer, void*, void*, void*, void*, void*, void*, void*,
                                                   void* g_normalized, int num_layers, int position, int cache_len,
                                                   int max_seq_len, float attn_scale, hipStream_t stream) {
  // the static workspace's tags cover at most MAX_LAYER_PASSES layers in one launch
  if (input_embedding == nullptr || num_layers < 1 || num_layers > qtts::MAX_LAYER_PASSES) return hipErrorInvalidValue;
  return ref_launch(true, 0, nullptr, input_embedding, layer_weights, final_norm_weight, cos_table, sin_table, k_cache,
                    v_cache, hidden_buffer, g_normalized, num_layers, position, cache_len, max_seq_len, attn_scale,
                    stream, /*static_ws=*/true);
}

hipError_t launch_cp_decode_with_embedding(const void* input_embedding, const CPLayerWeights* layer_weights,
                                           const void* final_norm_weight, const void* cos_table, const void* sin_table,
                                           void* k_cache, void* v_cache, void* hidden_buffer, void*, void*, void*,
                                           void*, void*, void*, void*, void* g_normalized, int num_layers,
                                           int position, int cache_len, int max_seq_len, float attn_scale,
                                           hipStream_t stream) {
  if (input_embedding == nullptr) return hipErrorInvalidValue;
  return ref_launch(false, 0, nullptr, input_embedding, layer_weights, final_norm_weight, cos_table, sin_table, k_cache,
                    v_cache, hidden_buffer, g_normalized, num_layers, position, cache_len, max_seq_len, attn_scale,
                    stream);
}

size_t qtts_workspace_bytes(void) { return sizeof(Workspace); }

hipError_t qtts_debug_trace(void* device_buffer, size_t bytes) {
  if (device_buffer != nullptr && bytes < (size_t)qtts::NWG * qtts::TRACE_STEPS * 2 * sizeof(uint64_t))
    return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lk(g_mu);
  g_trace = reinterpret_cast<uint64_t*>(device_buffer);
  return hipSuccess;
}

hipError_t qtts_workspace_init(void* workspace, int device) {
  if (workspace == nullptr || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return hipErrorInvalidValue;
  const hipError_t e = check_device(device);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_mu);
  g_seq.erase(workspace);   // new memory: the first launch that uses it zero-fills it
  return hipSuccess;
}

hipError_t qtts_workspace_release(void* workspace, int count) {
  if (workspace == nullptr || count < 1) return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lk(g_mu);
  for (int i = 0; i < count; ++i) g_seq.erase(reinterpret_cast<Workspace*>(workspace) + i);
  return hipSuccess;
}

hipError_t qtts_debug_set_sequence(void* workspace, unsigned int sequence) {
  if (workspace == nullptr || sequence < 1 || sequence > kSeqLimit) return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lk(g_mu);
  g_seq[workspace] = sequence;
  return hipSuccess;
}

hipError_t qtts_debug_set_error(void* workspace, unsigned int code, hipStream_t stream) {
  if (workspace == nullptr || code == 0u) return hipErrorInvalidValue;
  Workspace* ws = reinterpret_cast<Workspace*>(workspace);
  hipError_t e = hipMemcpyAsync(&ws->err, &code, sizeof(code), hipMemcpyHostToDevice, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  return e;
}

hipError_t qtts_debug_entry_spin_cap(unsigned int cap) {
  g_entry_cap.store(cap == 0u ? qtts_host::kEntrySpinCap : cap, std::memory_order_relaxed);
  return hipSuccess;
}

hipError_t qtts_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_seq.clear();
  g_trace = nullptr;
  if (g_lib_ws.empty() && g_dev.empty()) return hipSuccess;   // nothing on any device: no HIP call
  int cur = 0;
  hipError_t first = hipGetDevice(&cur);
  for (auto& kv : g_lib_ws) {
    if (kv.second == nullptr) continue;
    hipError_t e = hipSetDevice(kv.first.first);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipFree(kv.second);
    if (first == hipSuccess) first = e;
  }
  g_lib_ws.clear();
  g_seq.clear();
  g_trace = nullptr;
  for (auto& kv : g_dev) {
    if (kv.second.last == nullptr) continue;
    const hipError_t e = hipEventDestroy(kv.second.last);
    if (first == hipSuccess) first = e;
  }
  const bool any = !g_dev.empty();
  g_dev.clear();   // the next launch validates its device again
  if (any) {
    const hipError_t e = hipSetDevice(cur);
    if (first == hipSuccess) first = e;
  }
  return first;
}

hipError_t qtts_workspace_check(void* workspace, unsigned int* error_code, hipStream_t stream) {
  if (workspace == nullptr || error_code == nullptr) return hipErrorInvalidValue;
  Workspace* ws = reinterpret_cast<Workspace*>(workspace);
  hipError_t e = hipMemcpyAsync(error_code, &ws->err, sizeof(unsigned int), hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return e;
  if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
  if (*error_code != 0u) {
    unsigned int zero = 0u;
    e = hipMemcpy(&ws->err, &zero, sizeof(zero), hipMemcpyHostToDevice);
  }
  return e;
}

hipError_t qtts_backbone_step(void* workspace, const TTSLayerWeights* layer_weights, int num_layers,
                              const void* final_norm_weight, const void* cos_table, const void* sin_table,
                              void* k_cache, void* v_cache, int max_seq_len, int position, const int pos3[3],
                              const void* input_embedding, const void* embed_weight, int input_token_id,
                              float* out_hidden, void* out_residual, const void* codec_head, int vocab,
                              float* out_logits, int* out_token, int mask_tail, const int* history,
                              int n_history, float repetition_penalty, int eos_id, int suppress_eos,
                              const QttsSampling* sampling, int frame_step, const int* skip_if,
                              hipStream_t stream) {
  if (workspace == nullptr || (input_embedding == nullptr && embed_weight == nullptr)) return hipErrorInvalidValue;
  if (codec_head != nullptr && (vocab <= 0 || vocab > qtts::MAXV || vocab % (qtts::NWG * qtts::NMATH) != 0))
    return hipErrorInvalidValue;
  if (n_history < 0 || (n_history > 0 && history == nullptr)) return hipErrorInvalidValue;
  KArgs a;
  base_args(a, layer_weights, num_layers, final_norm_weight, cos_table, sin_table, k_cache, v_cache, max_seq_len);
  a.io[0].ws = reinterpret_cast<Workspace*>(workspace);
  a.io[0].pos0 = position;
  for (int i = 0; i < 3; ++i) a.io[0].pos3[i] = pos3 ? pos3[i] : position;
  for (int i = 0; i < 3; ++i)
    if (a.io[0].pos3[i] < 0 || a.io[0].pos3[i] >= max_seq_len) return hipErrorInvalidValue;
  a.io[0].in_emb = reinterpret_cast<const qtts::bf16_t*>(input_embedding);
  a.embed_w = reinterpret_cast<const qtts::bf16_t*>(embed_weight);
  a.io[0].in_tok = input_token_id;
  a.io[0].out_hidden = out_hidden;
  a.io[0].out_residual = out_residual;
  a.head = reinterpret_cast<const qtts::bf16_t*>(codec_head);
  a.vocab = vocab;
  a.io[0].out_logits = out_logits;
  a.io[0].out_token = out_token;
  a.mask_tail = mask_tail;
  a.io[0].skip = skip_if;
  a.io[0].history = history;
  a.io[0].n_history = n_history;
  a.rep_penalty = repetition_penalty;
  a.eos_id = eos_id;
  a.suppress_eos = suppress_eos;
  if (sampling) {
    a.sel.do_sample = sampling->do_sample;
    a.sel.temperature = sampling->temperature;
    a.sel.top_k = sampling->top_k;
    a.sel.top_p = sampling->top_p;
    a.io[0].seed = sampling->seed;
  }
  a.sel.frame_step = frame_step;
  return launch(true, a, stream);
}

hipError_t qtts_backbone_step_streams(int n_streams, void* workspaces, const TTSLayerWeights* layer_weights, int num_layers,
                                      const void* final_norm_weight, const void* cos_table, const void* sin_table,
                                      int max_seq_len, const QttsBackboneStream* streams, const void* codec_head, int vocab,
                                      int mask_tail, float repetition_penalty, int eos_id, int suppress_eos,
                                      const QttsSampling* sampling, int frame_step, hipStream_t stream) {
  if (n_streams < 1 || n_streams > qtts::NSTREAM || streams == nullptr) return hipErrorInvalidValue;
  if (workspaces == nullptr || (reinterpret_cast<uintptr_t>(workspaces) & 255u) != 0) return hipErrorInvalidValue;
  if (codec_head != nullptr && (vocab <= 0 || vocab > qtts::MAXV || vocab % (qtts::NWG * qtts::NMATH) != 0))
    return hipErrorInvalidValue;
  KArgs a;
  base_args(a, layer_weights, num_layers, final_norm_weight, cos_table, sin_table, nullptr, nullptr, max_seq_len);
  a.head = reinterpret_cast<const qtts::bf16_t*>(codec_head);
  a.vocab = vocab;
  a.mask_tail = mask_tail;
  a.rep_penalty = repetition_penalty;
  a.eos_id = eos_id;
  a.suppress_eos = suppress_eos;
  if (sampling) {
    a.sel.do_sample = sampling->do_sample;
    a.sel.temperature = sampling->temperature;
    a.sel.top_k = sampling->top_k;
    a.sel.top_p = sampling->top_p;
  }
  a.sel.frame_step = frame_step;
  for (int st = 0; st < n_streams; ++st) {
    const QttsBackboneStream& in = streams[st];
    if (in.k_cache == nullptr || in.v_cache == nullptr || in.input_embedding == nullptr) return hipErrorInvalidValue;
    if (in.position < 0 || in.position >= max_seq_len) return hipErrorInvalidValue;
    if (in.n_history < 0 || (in.n_history > 0 && in.history == nullptr)) return hipErrorInvalidValue;
    qtts::StreamIO& io = a.io[st];
    io.ws = reinterpret_cast<Workspace*>(workspaces) + st;
    io.kc = in.k_cache;
    io.vc = in.v_cache;
    io.pos0 = in.position;
    for (int i = 0; i < 3; ++i) {
      io.pos3[i] = in.pos3[i];
      if (io.pos3[i] < 0 || io.pos3[i] >= max_seq_len) return hipErrorInvalidValue;
    }
    io.in_emb = reinterpret_cast<const qtts::bf16_t*>(in.input_embedding);
    io.out_hidden = in.out_hidden;
    io.out_residual = in.out_residual;
    io.out_logits = in.out_logits;
    io.out_token = in.out_token;
    io.history = in.history;
    io.n_history = in.n_history;
    io.seed = in.seed;
    io.skip = in.skip_if;
  }
  // stream 0's position is the one launch() validates; the others were checked above
  return launch(true, a, stream, true, n_streams);
}

hipError_t qtts_cp_step(void* workspace, const CPLayerWeights* layer_weights, int num_layers,
                        const void* final_norm_weight, const void* cos_table, const void* sin_table, void* k_cache,
                        void* v_cache, int max_seq_len, int position, const void* input_embedding, float* out_hidden,
                        float* out_residual, hipStream_t stream) {
  if (workspace == nullptr || input_embedding == nullptr) return hipErrorInvalidValue;
  KArgs a;
  base_args(a, layer_weights, num_layers, final_norm_weight, cos_table, sin_table, k_cache, v_cache, max_seq_len);
  a.io[0].ws = reinterpret_cast<Workspace*>(workspace);
  a.io[0].pos0 = position;
  a.io[0].in_emb = reinterpret_cast<const qtts::bf16_t*>(input_embedding);
  a.io[0].out_hidden = out_hidden;
  a.io[0].out_residual = out_residual;
  return launch(false, a, stream);
}

hipError_t qtts_cp_frame(void* workspace, const CPLayerWeights* layer_weights, int num_layers,
                         const void* final_norm_weight, const void* cos_table, const void* sin_table, void* k_cache,
                         void* v_cache, int max_seq_len, const float* bb_hidden, const int* g0,
                         const void* bb_embedding, const void* const* lm_heads, const void* const* cp_embeddings,
                         int n_groups, int cp_vocab, const void* text_row, int* out_tokens, void* out_combined,
                         int* g0_history_slot, int eos_id, int* done, const QttsSampling* sampling, int frame_step,
                         hipStream_t stream) {
  if (workspace == nullptr || bb_hidden == nullptr || g0 == nullptr || bb_embedding == nullptr || lm_heads == nullptr ||
      cp_embeddings == nullptr || out_tokens == nullptr || out_combined == nullptr || done == nullptr)
    return hipErrorInvalidValue;
  if (n_groups < 1 || n_groups + 1 > 31 || n_groups + 1 > max_seq_len) return hipErrorInvalidValue;
  if (cp_vocab <= 0 || cp_vocab > qtts::MAXV || cp_vocab % (qtts::NWG * qtts::NMATH) != 0) return hipErrorInvalidValue;
  KArgs a;
  base_args(a, layer_weights, num_layers, final_norm_weight, cos_table, sin_table, k_cache, v_cache, max_seq_len);
  a.io[0].ws = reinterpret_cast<Workspace*>(workspace);
  a.io[0].pos0 = 0;
  a.n_pos = n_groups + 1;
  a.cp_frame = 1;
  a.io[0].bb_hidden = bb_hidden;
  a.io[0].g0 = g0;
  a.bb_emb = reinterpret_cast<const qtts::bf16_t*>(bb_embedding);
  a.cp_heads = reinterpret_cast<const qtts::bf16_t* const*>(lm_heads);
  a.cp_embs = reinterpret_cast<const qtts::bf16_t* const*>(cp_embeddings);
  a.n_groups = n_groups;
  a.cp_vocab = cp_vocab;
  a.io[0].text_row = reinterpret_cast<const qtts::bf16_t*>(text_row);
  a.io[0].out_tokens = out_tokens;
  a.io[0].hist_slot = g0_history_slot;
  a.io[0].out_combined = reinterpret_cast<qtts::bf16_t*>(out_combined);
  a.eos_id = eos_id;
  a.io[0].done = done;
  if (sampling) {
    a.sel.do_sample = sampling->do_sample;
    a.sel.temperature = sampling->temperature;
    a.sel.top_k = sampling->top_k;
    a.sel.top_p = sampling->top_p;
    a.io[0].seed = sampling->seed;
  }
  a.sel.frame_step = frame_step;
  return launch(false, a, stream);
}

hipError_t qtts_cp_frame_streams(int n_streams, void* workspaces, const CPLayerWeights* layer_weights, int num_layers,
                                 const void* final_norm_weight, const void* cos_table, const void* sin_table,
                                 void* k_caches, void* v_caches, int max_seq_len, const float* bb_hidden, const int* g0,
                                 const void* bb_embedding, const void* const* lm_heads, const void* const* cp_embeddings,
                                 int n_groups, int cp_vocab, const void* text_rows, int* out_tokens, void* out_combined,
                                 int eos_id, int* done, const QttsSampling* sampling, int frame_step, hipStream_t stream) {
  if (n_streams < 1 || n_streams > qtts::NSTREAM) return hipErrorInvalidValue;
  if (workspaces == nullptr || (reinterpret_cast<uintptr_t>(workspaces) & 255u) != 0 || k_caches == nullptr ||
      v_caches == nullptr || bb_hidden == nullptr || g0 == nullptr || bb_embedding == nullptr || lm_heads == nullptr ||
      cp_embeddings == nullptr || out_tokens == nullptr || out_combined == nullptr || done == nullptr)
    return hipErrorInvalidValue;
  // every position of the frame within one attention pass (the local path)
  if (n_groups < 1 || n_groups + 1 > qtts::KVGeo<false>::SUB || n_groups + 1 > max_seq_len) return hipErrorInvalidValue;
  if (cp_vocab <= 0 || cp_vocab > qtts::MAXV || cp_vocab % (qtts::NWG * qtts::NMATH) != 0) return hipErrorInvalidValue;
  KArgs a;
  base_args(a, layer_weights, num_layers, final_norm_weight, cos_table, sin_table, nullptr, nullptr, max_seq_len);
  a.n_pos = n_groups + 1;
  a.cp_frame = 1;
  a.bb_emb = reinterpret_cast<const qtts::bf16_t*>(bb_embedding);
  a.cp_heads = reinterpret_cast<const qtts::bf16_t* const*>(lm_heads);
  a.cp_embs = reinterpret_cast<const qtts::bf16_t* const*>(cp_embeddings);
  a.n_groups = n_groups;
  a.cp_vocab = cp_vocab;
  a.eos_id = eos_id;
  if (sampling) {
    a.sel.do_sample = sampling->do_sample;
    a.sel.temperature = sampling->temperature;
    a.sel.top_k = sampling->top_k;
    a.sel.top_p = sampling->top_p;
  }
  a.sel.frame_step = frame_step;
  const size_t kv = (size_t)num_layers * qtts::NKVH * (size_t)max_seq_len * qtts::HDIM;   // floats per stream
  for (int st = 0; st < n_streams; ++st) {
    qtts::StreamIO& io = a.io[st];
    io.ws = reinterpret_cast<Workspace*>(workspaces) + st;
    io.kc = reinterpret_cast<float*>(k_caches) + kv * st;
    io.vc = reinterpret_cast<float*>(v_caches) + kv * st;
    io.pos0 = 0;
    io.bb_hidden = bb_hidden + (size_t)qtts::HID * st;
    io.g0 = g0 + st;
    io.text_row = text_rows ? reinterpret_cast<const qtts::bf16_t*>(text_rows) + (size_t)qtts::HID * st : nullptr;
    io.out_tokens = out_tokens + (size_t)(n_groups + 1) * st;
    io.out_combined = reinterpret_cast<qtts::bf16_t*>(out_combined) + (size_t)qtts::HID * st;
    io.done = done + st;
    io.seed = sampling ? sampling->seed + (uint64_t)st : 0;
  }
  return launch(false, a, stream, true, n_streams);
}

}  // extern "C"
