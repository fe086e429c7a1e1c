// Weight-shared decode of several streams on MI355X (gfx950).
//
// One launch runs the backbone step (or the code-predictor frame) of up to 8 independent
// streams and reads every weight byte once for all of them: each workgroup applies its weight
// tile to the 8 streams' inputs at once with bf16 MFMA. The per-stream semantics are those of
// the batch-1 kernels (fused_decode_tts.cu:728-831, fused_decode_code_predictor.cu:565-668 and
// the frame glue of generator.py:116-174, 309-362); the reference itself decodes one stream.
//
// Decomposition: the batch-1 one. 256 workgroups, one per CU, tensor-parallel over the 8 XCDs
// (XCD x owns KV head x, query heads 2x and 2x+1, intermediate rows [384x, 384x+384) and the
// matching column slices of Wo and Wdown); inside an XCD the 32 workgroups split the rows
// (16 QKV, 32 O, 12 gate + 12 up, 32 down, 8 or 12 head rows each).
//
// Each workgroup has 8 waves; wave s does the vector work of stream slot s (its polls, norms,
// q/k-norm + RoPE, KV write, attention merge, token selection) and all 8 waves share the
// projections:
//   * The input of a projection is the 8 streams' f32 vectors, split exactly into three bf16
//     pieces (x = hi + mid + lo, hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid)),
//     kept in LDS. v_mfma_f32_16x16x32_bf16 multiplies a 16-row weight block by 16 columns
//     (hi and mid of the 8 streams) and a second one by the lo columns; the products are exact
//     and the sums are f32, so a projection carries f32 accuracy, as the reference's f32 GEMVs.
//   * The K dimension of a workgroup's tile is split over its waves; their partials meet in
//     LDS and are summed in a fixed order.
// Exchanges between workgroups use the tagged slots of the batch-1 kernels with a stream index
// added, so stream s of every step polls exactly the slots batch 1 would.
//
// Attention: the code predictor (at most 16 positions) attends locally in every workgroup,
// wave s over stream s. The backbone's ragged contexts are cut into 32 units per KV head
// (stream, chunk), sized by the host in proportion to the streams' lengths; workgroup li of an
// XCD takes unit li, its 8 waves split the unit's positions, and every workgroup merges the
// units of each stream when it forms that stream's O-projection input.
#include <hip/hip_runtime.h>
#include <atomic>
#include <cstddef>
#include <cstring>
#include <mutex>
#include <type_traits>
#include "qtts_common.h"
#include "qtts_host.h"
#include "qtts_poll.h"
#include "qtts_select.h"
#include "qwentts_amd.h"

namespace qtts {
namespace sh {

// Forced inlining for the kernel's lambdas: a real call passes the by-value launch arguments and
// the captured state by address, through scratch memory.
#define SH_INLINE __attribute__((always_inline))

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int NS = 8;                 // stream slots of a launch (one per wave)
constexpr int SWAV = 8;               // waves per workgroup
constexpr int STHR = 64 * SWAV;
constexpr int KP = HID + 8;           // bf16 row of one input column; the pad puts the 16 rows one
                                      // fragment read touches on distinct LDS banks
constexpr int XPS = 2 * NS * KP + 64; // bf16 elements from one input piece to the next (32 dwords past a
                                      // multiple of 64 banks: hi of stream s and mid of stream s, read
                                      // by one fragment, sit on distinct banks)
constexpr int NUNIT = WPX;            // attention units per KV head (one per workgroup)
constexpr int UMAX = 8;               // attention units of one stream
constexpr int UPH = 132;              // slots of one (unit, head) partial: acc[128], m, l, pad
constexpr int AJJ = 8;                // backbone attention: positions per lane group and pass
constexpr int APASS = 4 * AJJ * SWAV; // positions per workgroup pass
constexpr int CP_SUB = 16;            // code-predictor positions (one local pass)
constexpr uint32_t TAG_HEAD = 3584;   // head tags: TAG_HEAD + position
constexpr int MAX_LAYER_PASSES = 440;
constexpr double EPSD = (double)1e-6f;

enum TagSlot { T_QKV = 0, T_ATT, T_OPART, T_H1, T_INTER, T_DPART, T_XL, T_NSLOT = 8 };

// Exchange slots {f32 value, u32 tag}, double-buffered by layer-pass parity, with a stream index.
struct SWorkspace {
  uint64_t qkv[NXCD][2][NS][LROWS];
  uint64_t attp[NXCD][2][NUNIT][2][UPH];
  uint64_t h1[NXCD][2][NS][HID];
  uint64_t inter[NXCD][2][NS][XI];
  uint64_t xl[NXCD][2][NS][HID];
  uint64_t opart[2][NXCD][NS][HID];
  uint64_t dpart[2][NXCD][NS][HID];
  uint64_t logits[2][NS][MAXV];
  uint64_t hloc[NXCD][2][NS][2 * WPX];   // greedy CP heads: each workgroup's best {value, tag, id, tag}
  uint64_t hx[2][NS][WPX][2 * NXCD];     // every workgroup's copy of its XCD's best, [li][xcd]
  uint64_t tok[2][NS][2];                // sampled CP heads: the id selected for each stream
  uint32_t err;
  uint32_t pad[63];
};

struct SStream {
  void* kc;
  void* vc;
  int pos;                 // backbone: cache slot of the new token (attention covers 0..pos)
  int pos3[3];             // backbone: rotary (t, h, w)
  const bf16_t* in_emb;
  float* out_hidden;
  void* out_residual;
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
  bf16_t* out_combined;
  int* done;
  uint64_t seed;
  // backbone attention: units u0 .. u0 + nu - 1 (workgroup li of each XCD takes unit li), P positions each
  int u0, nu, P;
};

struct SArgs {
  SWorkspace* ws;
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
  int n_pos;
  int n_streams;
  const bf16_t* head;
  int vocab;
  int mask_tail;
  float rep_penalty;
  int eos_id;
  int suppress_eos;
  int cp_frame;
  const bf16_t* bb_emb;
  const bf16_t* const* cp_heads;
  const bf16_t* const* cp_embs;
  int n_groups;
  int cp_vocab;
  SelParams sel;
  int unit_stream[NUNIT];  // stream of attention unit u, -1 for none
  uint64_t* trace;         // optional step timeline: [wg][step][TRACE_SLOTS] s_memrealtime stamps
  SStream io[NS];
};
// timeline slots of a step: 0 after the entry barrier, 1 after the partials barrier, 2 + w the
// end of wave w's vector work, 10 .. 15 points inside the step (wave 0)
constexpr int TRACE_SLOTS = 16;
constexpr int TRACE_STEPS = 1024;

struct SLds {
  union {
    // projection input pieces (hi, mid, lo): piece p of column n at xb[p * XPS + n * KP]. Columns
    // 0..7 are the streams; the code-predictor frame's two-column pass puts position 1 of
    // stream s in column 8 + s
    alignas(16) bf16_t xb[3 * XPS];
    struct {
      alignas(16) float stage[MAXV];    // token selection of one stream (its own workgroup)
      SelScratch sel;
    } z;
  };
  alignas(16) float red[SWAV][16][2 * NS];   // per wave: its K-slice's partial of 16 rows x 16 columns
  alignas(16) float q[NS][2][HDIM];
  alignas(16) float knew[NS][HDIM];
  alignas(16) float vnew[NS][HDIM];
  float wpart[SWAV][2][HDIM + 2];       // backbone attention: per wave (acc, m, l) of each head
  float xres[NS][32];                   // the workgroup's 32 rows of each stream's residual x ...
  float h1res[NS][32];                  // ... and of h1
  float xres1[NS][32];                  // the same of position 1 in the two-column pass
  float h1res1[NS][32];
  alignas(16) float comb[HID];          // CP frame: running combine of this workgroup's stream
  const bf16_t* embp[16];
  int tok[NS][16];
  uint32_t pen_bits[NS][MAXV / 32];
};

struct TQ { u32x4 p[4]; };   // QKV / head: 4 K-blocks of the wave
struct TO { u32x4 p[2]; };
struct TG { u32x4 p[8]; };
struct TD { u32x4 p[3]; };
struct TKV { u32x4 k[AJJ]; u32x4 v[AJJ]; };

enum { W_LNIN = 0, W_Q, W_K, W_V, W_QN, W_KN, W_O, W_LNPOST, W_GATE, W_UP, W_DOWN };
__device__ __forceinline__ const bf16_t* lw(const TTSLayerWeights* layers, int layer, int i) {
  const void* const* p = reinterpret_cast<const void* const*>(layers + layer);
  return reinterpret_cast<const bf16_t*>(ld_const(p + i));
}
__device__ __forceinline__ bf16x8 as_bf8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
// the value of lane (lane ^ 8) within each 16-lane row
__device__ __forceinline__ float ror8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
}
// exact three-piece bf16 split of two values, as packed pairs: x = hi + mid + lo up to 2^-24 |x|
// (each residual is exact in f32); the conversion instruction rounds to nearest even, three per
// pair instead of about forty for the bit-manipulation rounding
__device__ __forceinline__ void split3x2(float x0, float x1, uint32_t& h, uint32_t& m, uint32_t& l) {
  h = f2bf2(x0, x1);
  const float r0 = x0 - bflo(h), r1 = x1 - bfhi(h);
  m = f2bf2(r0, r1);
  l = f2bf2(r0 - bflo(m), r1 - bfhi(m));
}

// Sum of the 8 XCD partials of rows r0 + 2 (lane & 15) + {0, 1} of one stream: lane group
// g = lane >> 4 polls XCDs 2 g and 2 g + 1; two exchanges complete the sum as
// ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)), the same in every lane and workgroup.
// p0 points at XCD 0's slot of row r0; consecutive XCDs are NS * HID slots apart.
__device__ __forceinline__ bool poll_sum8s(const Poll& P, const uint64_t* p0, uint32_t tag, double& s0, double& s1) {
  const uint32_t o = ws_off(P, p0);
  float v[4];
  const bool ok = poll_regs<2>(P, 128, tag, v, [o](int i) {
    const uint32_t x = 2u * (uint32_t)((i & 63) >> 4) + (uint32_t)(i >> 6);
    return o + x * (uint32_t)(NS * HID * 8) + 16u * (uint32_t)(i & 15);
  });
  s0 = (double)v[0] + (double)v[2];
  s1 = (double)v[1] + (double)v[3];
  s0 += xlane_d<4>(s0);
  s1 += xlane_d<4>(s1);
  s0 += xlane_d<5>(s0);
  s1 += xlane_d<5>(s1);
  return ok;
}


// Token selection over an LDS logit vector, kept out of line: inlined, the loop-invariant parts of
// its sampler would be hoisted out of the step loops and hold registers (or spill) for the whole
// launch; it runs at most once per head.
__device__ __attribute__((noinline)) int sh_wave_select(const float* lg, int n, SelParams sp, SelScratch* sc) {
  return wave_select(lg, n, sp, sc);
}

template <bool BB>
__global__ void __launch_bounds__(STHR, 1) qtts_shared_kernel(const SArgs a) {
  __shared__ SLds s;
  // norm statistics in f64 for the backbone (its bf16 residual), f32 in the code predictor
  // norms and their sums in f32 for both models: the projections already sum in f32 (MFMA), so
  // the batch-1 backbone's f64 norms would buy no accuracy here, only VALU time and registers
  using A = float;
  // lane and thread index, re-derived opaquely at every step so that offsets computed from them
  // are recomputed where used instead of being hoisted out of the step loop and spilled
  int lane = threadIdx.x & 63;
  int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));   // wave = stream slot
  const int xcd = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u);   // HW_REG_XCC_ID
  const int li = blockIdx.x >> 3;
  const int wg = blockIdx.x;
  // per-stream blocks read through the kernel-argument segment (uniform offsets: scalar loads;
  // indexing the by-value argument with a run-time index would copy it to scratch)
  typedef const __attribute__((address_space(4))) SStream* IOP;
  const IOP IO0 = (IOP)((const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr() +
                        offsetof(SArgs, io));
  const IOP IO = IO0 + wv;
  SWorkspace* ws = a.ws;
  const TTSLayerWeights* LW = a.layers;
  const int NL = a.num_layers;
  const bool cp = a.cp_frame != 0;
  const bool cp_greedy = cp && !a.sel.do_sample;

  // streams that compute in this launch (the same set in every workgroup): not skipped, and in
  // a code-predictor frame not already at EOS (generator.py:124-125; its done flag is set)
  uint32_t live = 0;
  for (int t = 0; t < a.n_streams; ++t) {
    const IOP io = IO0 + t;
    bool on = io->skip == nullptr || *io->skip == 0;
    if (on && cp && a.eos_id >= 0 && *io->g0 == a.eos_id) {
      on = false;
      if (wg == 0 && threadIdx.x == 0) *io->done = 1;
    }
    if (on) live |= 1u << t;
  }
  if (live == 0u) return;
  const bool me = (live >> wv) & 1u;   // this wave's stream computes
  auto is_live = [&](int t) { return ((live >> t) & 1u) != 0u; };

  // projection inputs start at zero: a stream that computes nothing keeps finite columns
  for (int i = threadIdx.x; i < (int)(sizeof(s.xb) / 16); i += STHR)
    reinterpret_cast<u32x4*>(&s.xb[0])[i] = u32x4{0u, 0u, 0u, 0u};
  if (cp && (int)threadIdx.x < a.n_groups) s.embp[threadIdx.x] = a.cp_embs[threadIdx.x];
  __syncthreads();

  Poll P;
  P.rs = __builtin_amdgcn_make_buffer_rsrc(ws, (short)0, (int)sizeof(SWorkspace), 0x00020000);
  P.base = ws;
  P.ec.err = &ws->err;
  // the first layer pass waits under the short entry cap (an arrival check: its exchanges need
  // every workgroup of the launch); the long cap from the second pass on
  P.ec.spin_cap = a.entry_spin_cap;
  // slot publishes: XCD-local as plain stores (they land in the XCD's L2), cross-XCD with sc1
  // (written through to memory); one store carries value and tag together
  auto pub_local = [&](const uint64_t* p, float v, uint32_t tag) {
    const u32x2 d = {__float_as_uint(v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(d, P.rs, (int)ws_off(P, p), 0, 0);
  };
  auto pub_cross = [&](const uint64_t* p, float v, uint32_t tag) {
    const u32x2 d = {__float_as_uint(v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(d, P.rs, (int)ws_off(P, p), 0, 16);
  };
  auto pub_local2 = [&](const uint64_t* p, float v0, float v1, uint32_t tag) {
    const u32x4 d = {__float_as_uint(v0), tag, __float_as_uint(v1), tag};
    __builtin_amdgcn_raw_buffer_store_b128(d, P.rs, (int)ws_off(P, p), 0, 0);
  };
  auto tag_of = [&](int lp, int slot) -> uint32_t { return a.tag_base + (uint32_t)(lp * T_NSLOT + slot); };
  int nstep = 0;
  auto stamp = [&](int slot) {
    if (a.trace != nullptr && lane == 0 && nstep < TRACE_STEPS && ((slot >= 2 && slot < 2 + SWAV) || wv == 0))
      a.trace[((size_t)wg * TRACE_STEPS + nstep) * TRACE_SLOTS + slot] = __builtin_amdgcn_s_memrealtime();
  };
  auto has_head = [&](int pi) -> bool { return cp ? pi >= 1 : (a.head != nullptr && pi == a.n_pos - 1); };

  // ---- per-wave vectors of its stream: RMSNorm gains of the lane's 16 hidden elements
  // 2 (lane + 64 k) + {0, 1}, q/k-norm gains and rotary of head channels lane, lane + 64
  uint32_t gp[8];
  float qn[2], kn[2], rc[2], rsn[2];
  auto load_gains = [&](const bf16_t* src) {
    const auto* p = gmem(reinterpret_cast<const uint32_t*>(src));
#pragma unroll
    for (int k = 0; k < 8; ++k) gp[k] = p[lane + 64 * k];
  };
  auto rot_row = [&](int c, int pos) -> int {
    if constexpr (BB) {
      const int sec = (c < 60 && c % 3 == 1) ? 1 : ((c < 60 && c % 3 == 2) ? 2 : 0);
      return IO->pos3[sec];
    } else {
      return pos;
    }
  };
  auto load_qk = [&](int layer, int pos) {
    const bf16_t* q = lw(LW, layer, W_QN);
    const bf16_t* k = lw(LW, layer, W_KN);
    qn[0] = ldbf(q + lane); qn[1] = ldbf(q + lane + 64);
    kn[0] = ldbf(k + lane); kn[1] = ldbf(k + lane + 64);
    const size_t row = (size_t)rot_row(lane, pos) * HDIM;   // channel lane + 64 shares the row
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      rc[j] = ldbf(a.cos_t + row + lane + 64 * j);
      rsn[j] = ldbf(a.sin_t + row + lane + 64 * j);
    }
  };
  // f32((x * rstd) * g) of the lane's 16 elements, rstd = 1 / sqrt(mean(x^2) + eps)
  auto normed = [&](const float (&xv)[16], float (&y)[16]) {
    A s4[4] = {A(0), A(0), A(0), A(0)};
#pragma unroll
    for (int j = 0; j < 16; ++j) s4[j & 3] = fma((A)xv[j], (A)xv[j], s4[j & 3]);
    const A ss = group_sum<64>((s4[0] + s4[1]) + (s4[2] + s4[3]));
    const A r = rsqrt_a(ss / (A)HID + (A)EPSD);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      y[2 * k] = (float)(((A)xv[2 * k] * r) * (A)bflo(gp[k]));
      y[2 * k + 1] = (float)(((A)xv[2 * k + 1] * r) * (A)bfhi(gp[k]));
    }
  };
  // projection input column n: elements e, e + 1 of its three pieces
  auto put_pair_n = [&](int n, int e, float v0, float v1) {
    uint32_t h, m, l;
    split3x2(v0, v1, h, m, l);
    *reinterpret_cast<uint32_t*>(&s.xb[n * KP + e]) = h;
    *reinterpret_cast<uint32_t*>(&s.xb[XPS + n * KP + e]) = m;
    *reinterpret_cast<uint32_t*>(&s.xb[2 * XPS + n * KP + e]) = l;
  };
  // element e alone
  auto put_one_n = [&](int n, int e, float v) {
    uint32_t h, m, l;
    split3x2(v, 0.0f, h, m, l);
    s.xb[n * KP + e] = (bf16_t)h;
    s.xb[XPS + n * KP + e] = (bf16_t)m;
    s.xb[2 * XPS + n * KP + e] = (bf16_t)l;
  };
  // this wave's stream (column wv)
  auto put_pair = [&](int e, float v0, float v1) { put_pair_n(wv, e, v0, v1); };
  auto put_vec_n = [&](int n, const float (&y)[16]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) put_pair_n(n, 2 * (lane + 64 * k), y[2 * k], y[2 * k + 1]);
  };
  auto put_vec = [&](const float (&y)[16]) { put_vec_n(wv, y); };
  // the workgroup's 32 rows 32 li + m of a lane-distributed vector: lanes 16 (li & 3) .. + 15
  // hold them at k = li >> 2
  auto keep_rows = [&](float* dst, const float (&xv)[16]) {
    // a select chain over k (a uniform index into the register array would go through scratch)
    const int kk = li >> 2;
    float v0 = xv[0], v1 = xv[1];
#pragma unroll
    for (int k = 1; k < 8; ++k) {
      v0 = k == kk ? xv[2 * k] : v0;
      v1 = k == kk ? xv[2 * k + 1] : v1;
    }
    if ((lane >> 4) == (li & 3)) *reinterpret_cast<float2*>(&dst[2 * (lane & 15)]) = make_float2(v0, v1);
  };

  // ---- vector work of this wave's stream --------------------------------------------------
  // input of layer 0 at position pi; the code-predictor frame's combine accumulates the inputs
  // of positions 1.. in the stream's own workgroup (bf16 rounding after each add, in the order
  // emb_bb[g0] + emb_0[t_0] + ...; generator.py:356-362)
  auto prep_input0 = [&](int pi, int n, float* keep) {
    load_gains(lw(LW, 0, W_LNIN));
    float xv[16];
    if (cp && pi == 0) {
      const auto* p = gmem(reinterpret_cast<const u32x2*>(IO->bb_hidden));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const u32x2 v = p[lane + 64 * k];
        xv[2 * k] = rbf(__uint_as_float(v.x));
        xv[2 * k + 1] = rbf(__uint_as_float(v.y));
      }
    } else {
      const bf16_t* src = cp ? (pi == 1 ? a.bb_emb + (size_t)(*IO->g0) * HID : s.embp[pi - 2] + (size_t)s.tok[wv][pi - 2] * HID)
                             : IO->in_emb;
      const auto* p = gmem(reinterpret_cast<const uint32_t*>(src));
#pragma unroll
      for (int k = 0; k < 8; ++k) { const uint32_t w = p[lane + 64 * k]; xv[2 * k] = bflo(w); xv[2 * k + 1] = bfhi(w); }
    }
    keep_rows(keep, xv);
    if (cp && pi >= 1 && wg == wv) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = 2 * (lane + 64 * k);
        const float2 c = *reinterpret_cast<const float2*>(&s.comb[e]);
        *reinterpret_cast<float2*>(&s.comb[e]) = pi == 1 ? make_float2(xv[2 * k], xv[2 * k + 1])
                                                         : make_float2(rbf(c.x + xv[2 * k]), rbf(c.y + xv[2 * k + 1]));
      }
    }
    float y[16];
    normed(xv, y);
    put_vec_n(n, y);
  };
  // q/k norm, RoPE and the KV write of layer `layer` at cache slot pos. The lane holds channels
  // c = lane and c + 64 (the rotate_half partners) of q head 0, q head 1, k and v.
  bool kv_pending = false;
  auto prep_att = [&](int lp, int layer, int pos, auto&& issue) SH_INLINE {
    load_qk(layer, pos);
    float v[8];
    {
      const uint32_t o = ws_off(P, &ws->qkv[xcd][lp & 1][wv][0]);
      poll_regs<4>(P, LROWS / 2, tag_of(lp, T_QKV), v, [o](int i) { return o + 16u * (uint32_t)i; });
    }
    issue();
    A ss[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) ss[h] = fma((A)v[2 * h], (A)v[2 * h], (A)v[2 * h + 1] * (A)v[2 * h + 1]);
    group_sum_n<64, 3>(ss);
    const A cl = rc[0], ch = rc[1], sl = rsn[0], sh_ = rsn[1];
    float outl[3], outh[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      const A r = rsqrt_a(ss[h] / (A)HDIM + (A)EPSD);
      const A gl = h < 2 ? qn[0] : kn[0], gh = h < 2 ? qn[1] : kn[1];
      const A nl = ((A)v[2 * h] * r) * gl, nh = ((A)v[2 * h + 1] * r) * gh;
      outl[h] = (float)(nl * cl - nh * sl);
      outh[h] = (float)(nl * sh_ + nh * ch);
    }
    const int c = lane;
    s.q[wv][0][c] = outl[0]; s.q[wv][0][c + 64] = outh[0];
    s.q[wv][1][c] = outl[1]; s.q[wv][1][c + 64] = outh[1];
    float kl = outl[2], kh = outh[2], vl = v[6], vh = v[7];
    if constexpr (BB) { kl = rbf(kl); kh = rbf(kh); vl = rbf(vl); vh = rbf(vh); }
    s.knew[wv][c] = kl; s.knew[wv][c + 64] = kh;
    s.vnew[wv][c] = vl; s.vnew[wv][c + 64] = vh;
    if (li == 0) {
      const size_t off = (((size_t)layer * NKVH + xcd) * (size_t)a.max_seq + pos) * HDIM + c;
      if constexpr (BB) {
        bf16_t* kc = reinterpret_cast<bf16_t*>(IO->kc) + off;
        bf16_t* vc = reinterpret_cast<bf16_t*>(IO->vc) + off;
        gput(kc, f2bf(kl)); gput(kc + 64, f2bf(kh));
        gput(vc, f2bf(vl)); gput(vc + 64, f2bf(vh));
      } else {
        float* kc = reinterpret_cast<float*>(IO->kc) + off;
        float* vc = reinterpret_cast<float*>(IO->vc) + off;
        gput(kc, kl); gput(kc + 64, kh);
        gput(vc, vl); gput(vc + 64, vh);
        // read at later positions of this launch by the XCD's workgroups (through its L2):
        // complete before this wave's next slot publish (ar1)
        kv_pending = true;
      }
    }
  };
  // the stream's O-projection input: merge of its attention units (backbone). Lane (h, dq):
  // head h = lane >> 5, dims dq .. dq + 3 (dq = 4 (lane & 31)). First the (m, l) pair of head h
  // of every unit: w_c = exp(m_c - M), Z = sum_c w_c l_c; then two acc pairs per unit:
  // out = (sum_c w_c acc_c) / Z. (Two polls keep fewer registers live than one.)
  auto prep_o = [&](int lp) SH_INLINE {
    const int u0 = IO->u0, nu = IO->nu;
    const int h = lane >> 5, dq = 4 * (lane & 31);
    const uint32_t o = ws_off(P, &ws->attp[xcd][lp & 1][0][0][0]);
    const uint32_t tg = tag_of(lp, T_ATT);
    float w[UMAX];
    float Z = 0.0f;
    {
      float ml[2 * UMAX];
      poll_regs<UMAX>(P, 64 * nu, tg, ml, [o, u0](int i) {
        const uint32_t c = (uint32_t)i >> 6, l = (uint32_t)i & 63u;
        return o + 8u * ((((uint32_t)u0 + c) * 2u + (l >> 5)) * (uint32_t)UPH + 128u);
      });
      float M = -INFINITY;
#pragma unroll
      for (int c = 0; c < UMAX; ++c)
        if (c < nu) M = fmaxf(M, ml[2 * c]);
#pragma unroll
      for (int c = 0; c < UMAX; ++c) {
        // slots c >= nu were never polled: their registers are not read (garbage times 0 can be NaN)
        w[c] = c < nu ? __expf(ml[2 * c] - M) : 0.0f;
        Z = fmaf(c < nu ? ml[2 * c + 1] : 0.0f, w[c], Z);
      }
    }
    float acc[2 * 2 * UMAX];
    read_pairs<2 * UMAX>(P, 64 * 2 * nu, tg, acc, [o, u0](int i) {
      const uint32_t k = (uint32_t)i >> 6, l = (uint32_t)i & 63u, c = k >> 1;
      return o + 8u * ((((uint32_t)u0 + c) * 2u + (l >> 5)) * (uint32_t)UPH + 4u * (l & 31u) + 2u * (k & 1u));
    });
    float o4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < UMAX; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) o4[j] = fmaf(c < nu ? acc[4 * c + j] : 0.0f, w[c], o4[j]);
    const float rz = rcp_f(Z);
    put_pair(128 * h + dq, o4[0] * rz, o4[1] * rz);
    put_pair(128 * h + dq + 2, o4[2] * rz, o4[3] * rz);
  };
  // AR1: h1 = x + the sum of the 8 XCD O partials, rows 32 li .. + 31 of this stream
  // (lp: the layer pass whose tags are used, par: the buffer, xr: the residual rows)
  auto ar1 = [&](int lp, int par, const float* xr) {
    const int r2 = 2 * (lane & 15);
    const float r0 = xr[r2], r1 = xr[r2 + 1];
    double s0, s1;
    poll_sum8s(P, &ws->opart[par][0][wv][32 * li], tag_of(lp, T_OPART), s0, s1);
    if (kv_pending) {
      // the KV entry written in prep_att: its stores complete before this publish
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      kv_pending = false;
    }
    if (lane < 16)
      pub_local2(&ws->h1[xcd][par][wv][32 * li + r2], (float)((double)r0 + s0), (float)((double)r1 + s1), tag_of(lp, T_H1));
  };
  // AR2: x' = h1 + the sum of the 8 XCD down partials (bf16 residual in the backbone)
  auto ar2 = [&](int lp, int par, const float* hr) {
    const int r2 = 2 * (lane & 15);
    const float r0 = hr[r2], r1 = hr[r2 + 1];
    double s0, s1;
    poll_sum8s(P, &ws->dpart[par][0][wv][32 * li], tag_of(lp, T_DPART), s0, s1);
    if (lane < 16) {
      float x0 = (float)((double)r0 + s0), x1 = (float)((double)r1 + s1);
      if constexpr (BB) { x0 = rbf(x0); x1 = rbf(x1); }
      pub_local2(&ws->xl[xcd][par][wv][32 * li + r2], x0, x1, tag_of(lp, T_XL));
    }
  };
  // final norm: outputs (the stream's own workgroup) and the head input bf16(h)
  auto prep_final = [&](int lp) {
    load_gains(a.final_norm);
    float xv[16], y[16];
    gather1024(P, &ws->xl[xcd][lp & 1][wv][0], tag_of(lp, T_XL), xv);
    normed(xv, y);
    if (wg == wv) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = 2 * (lane + 64 * k);
        if (IO->out_hidden) *reinterpret_cast<float2*>(IO->out_hidden + e) = make_float2(y[2 * k], y[2 * k + 1]);
        if (IO->out_residual) {
          if constexpr (BB)
            reinterpret_cast<uint32_t*>(IO->out_residual)[e >> 1] =
                (uint32_t)f2bf(xv[2 * k]) | ((uint32_t)f2bf(xv[2 * k + 1]) << 16);
          else
            *reinterpret_cast<float2*>(reinterpret_cast<float*>(IO->out_residual) + e) = make_float2(xv[2 * k], xv[2 * k + 1]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) y[j] = rbf(y[j]);
    put_vec(y);
  };

  // These vector phases take the issue of the next step's weight tile as an argument and make it
  // right after their last poll: a wave's vector-memory results return in issue order, so a poll
  // issued behind a tile load waits for the tile's HBM round trip. Both models use them for the
  // QKV, O, gate/up and (except after the last layer) down steps; the code predictor also for
  // its inputs and final norm.
  auto cp_prep_input0 = [&](int pi, auto&& issue) SH_INLINE {
    load_gains(lw(LW, 0, W_LNIN));
    float xv[16];
    if (pi == 0) {
      const auto* p = gmem(reinterpret_cast<const u32x2*>(IO->bb_hidden));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const u32x2 v = p[lane + 64 * k];
        xv[2 * k] = rbf(__uint_as_float(v.x));
        xv[2 * k + 1] = rbf(__uint_as_float(v.y));
      }
    } else {
      const bf16_t* src = pi == 1 ? a.bb_emb + (size_t)(*IO->g0) * HID : s.embp[pi - 2] + (size_t)s.tok[wv][pi - 2] * HID;
      const auto* p = gmem(reinterpret_cast<const uint32_t*>(src));
#pragma unroll
      for (int k = 0; k < 8; ++k) { const uint32_t w = p[lane + 64 * k]; xv[2 * k] = bflo(w); xv[2 * k + 1] = bfhi(w); }
    }
    issue();
    keep_rows(s.xres[wv], xv);
    if (pi >= 1 && wg == wv) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = 2 * (lane + 64 * k);
        const float2 c = *reinterpret_cast<const float2*>(&s.comb[e]);
        *reinterpret_cast<float2*>(&s.comb[e]) = pi == 1 ? make_float2(xv[2 * k], xv[2 * k + 1])
                                                         : make_float2(rbf(c.x + xv[2 * k]), rbf(c.y + xv[2 * k + 1]));
      }
    }
    float y[16];
    normed(xv, y);
    put_vec(y);
  };
  auto cp_prep_att = [&](int lp, int layer, int pos, auto&& issue) SH_INLINE {
    load_qk(layer, pos);
    float v[8];
    {
      const uint32_t o = ws_off(P, &ws->qkv[xcd][lp & 1][wv][0]);
      poll_regs<4>(P, LROWS / 2, tag_of(lp, T_QKV), v, [o](int i) { return o + 16u * (uint32_t)i; });
    }
    issue();
    float ss[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) ss[h] = fmaf(v[2 * h], v[2 * h], v[2 * h + 1] * v[2 * h + 1]);
    group_sum_n<64, 3>(ss);
    float outl[3], outh[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      const float r = rsqrt_a(ss[h] / (float)HDIM + (float)EPSD);
      const float gl = h < 2 ? qn[0] : kn[0], gh = h < 2 ? qn[1] : kn[1];
      const float nl = (v[2 * h] * r) * gl, nh = (v[2 * h + 1] * r) * gh;
      outl[h] = nl * rc[0] - nh * rsn[0];
      outh[h] = nl * rsn[1] + nh * rc[1];
    }
    const int c = lane;
    s.q[wv][0][c] = outl[0]; s.q[wv][0][c + 64] = outh[0];
    s.q[wv][1][c] = outl[1]; s.q[wv][1][c + 64] = outh[1];
    s.knew[wv][c] = outl[2]; s.knew[wv][c + 64] = outh[2];
    s.vnew[wv][c] = v[6]; s.vnew[wv][c + 64] = v[7];
    if (li == 0) {
      float* kc = reinterpret_cast<float*>(IO->kc) + (((size_t)layer * NKVH + xcd) * (size_t)a.max_seq + pos) * HDIM + c;
      float* vc = reinterpret_cast<float*>(IO->vc) + (((size_t)layer * NKVH + xcd) * (size_t)a.max_seq + pos) * HDIM + c;
      gput(kc, outl[2]); gput(kc + 64, outh[2]);
      gput(vc, v[6]); gput(vc + 64, v[7]);
      kv_pending = true;   // ordered before this wave's next slot publish (ar1)
    }
  };
  // a gathered 1024-vector (h1 or the residual after the down projection): its norm into projection
  // input column n, the workgroup's rows kept in `keep`; `issue` runs after the gather's last poll,
  // `issue2` after the vector work
  auto cp_prep_vec2 = [&](const uint64_t* base, uint32_t tag, const bf16_t* gains, float* keep, int n, auto&& issue, auto&& issue2) SH_INLINE {
    load_gains(gains);
    float xv[16], y[16];
    gather1024(P, base, tag, xv);
    issue();
    keep_rows(keep, xv);
    normed(xv, y);
    put_vec_n(n, y);
    issue2();
  };
  auto cp_prep_vec = [&](const uint64_t* base, uint32_t tag, const bf16_t* gains, float* keep, int n, auto&& issue) SH_INLINE {
    cp_prep_vec2(base, tag, gains, keep, n, issue, []() SH_INLINE {});
  };
  auto cp_prep_down = [&](int lp, auto&& issue) SH_INLINE {
    float v[6];
    const uint32_t o = ws_off(P, &ws->inter[xcd][lp & 1][wv][0]);
    poll_regs<3>(P, XI / 2, tag_of(lp, T_INTER), v, [o](int i) { return o + 16u * (uint32_t)i; });
    issue();
#pragma unroll
    for (int k = 0; k < 3; ++k) put_pair(2 * (lane + 64 * k), v[2 * k], v[2 * k + 1]);
  };
  auto cp_prep_final = [&](int lp, int par, auto&& issue) SH_INLINE {
    load_gains(a.final_norm);
    float xv[16];
    gather1024(P, &ws->xl[xcd][par][wv][0], tag_of(lp, T_XL), xv);
    issue();
    float y[16];
    normed(xv, y);
    if (wg == wv) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = 2 * (lane + 64 * k);
        if (IO->out_hidden) *reinterpret_cast<float2*>(IO->out_hidden + e) = make_float2(y[2 * k], y[2 * k + 1]);
        if (IO->out_residual)
          *reinterpret_cast<float2*>(reinterpret_cast<float*>(IO->out_residual) + e) = make_float2(xv[2 * k], xv[2 * k + 1]);
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) y[j] = rbf(y[j]);
    put_vec(y);
  };

  // ---- two-column pass of the code-predictor frame -------------------------------------------
  // Positions 0 and 1 of every stream (generator.py:318-344 runs them as a 2-token prefill) share
  // one pass over the weights: both inputs are known at launch (bf16(h) and emb_bb[g0]) and
  // position 1's layer l attends to position 0's layer-l entry and its own. Column wv of the
  // projection inputs carries position 0, column NS + wv position 1. Both columns of layer l
  // publish with layer pass l's tags, column c into buffer parity (l & 1) ^ c, so that one poll
  // covers both (by the exchange chain, every reader of a buffer is done before the next step's
  // writers reach it). Position 0's last layer only writes its K/V entry.
  auto dpar = [&](int layer, int c) { return (layer & 1) ^ c; };
  // q/k norm + RoPE and the KV write of both positions, then position 1's attention over the two
  // entries, in registers (lane: channels c = lane and c + 64 of each head block); position 0's
  // attention output is its own v (one entry, weight exactly 1)
  auto duo_prep_att = [&](int layer, auto&& issue) SH_INLINE {
    load_qk(layer, 0);
    float rc1[2], rsn1[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      rc1[j] = ldbf(a.cos_t + HDIM + lane + 64 * j);
      rsn1[j] = ldbf(a.sin_t + HDIM + lane + 64 * j);
    }
    float v[16];   // position c: v[8 c + 2 b + {0, 1}] = channels c, c + 64 of block b (q0, q1, k, v)
    {
      const uint32_t o0 = ws_off(P, &ws->qkv[xcd][dpar(layer, 0)][wv][0]);
      const uint32_t o1 = ws_off(P, &ws->qkv[xcd][dpar(layer, 1)][wv][0]);
      poll_regs<8>(P, LROWS, tag_of(layer, T_QKV), v, [o0, o1](int i) {
        return i < LROWS / 2 ? o0 + 16u * (uint32_t)i : o1 + 16u * (uint32_t)(i - LROWS / 2);
      });
    }
    issue();
    // norm statistics: position 0's k; position 1's q0, q1, k
    float ss[4];
    ss[0] = fmaf(v[4], v[4], v[5] * v[5]);
#pragma unroll
    for (int h = 0; h < 3; ++h) ss[1 + h] = fmaf(v[8 + 2 * h], v[8 + 2 * h], v[9 + 2 * h] * v[9 + 2 * h]);
    group_sum_n<64>(ss);
    float k0l, k0h;
    {
      const float r = rsqrt_a(ss[0] / (float)HDIM + (float)EPSD);
      const float nl = (v[4] * r) * kn[0], nh = (v[5] * r) * kn[1];
      k0l = nl * rc[0] - nh * rsn[0];
      k0h = nl * rsn[1] + nh * rc[1];
    }
    float outl[3], outh[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      const float r = rsqrt_a(ss[1 + h] / (float)HDIM + (float)EPSD);
      const float gl = h < 2 ? qn[0] : kn[0], gh = h < 2 ? qn[1] : kn[1];
      const float nl = (v[8 + 2 * h] * r) * gl, nh = (v[9 + 2 * h] * r) * gh;
      outl[h] = nl * rc1[0] - nh * rsn1[0];
      outh[h] = nl * rsn1[1] + nh * rc1[1];
    }
    const int c = lane;
    if (li == 0) {
      const size_t e0 = (((size_t)layer * NKVH + xcd) * (size_t)a.max_seq) * HDIM + c;
      float* kc = reinterpret_cast<float*>(IO->kc) + e0;
      float* vc = reinterpret_cast<float*>(IO->vc) + e0;
      gput(kc, k0l); gput(kc + 64, k0h);
      gput(vc, v[6]); gput(vc + 64, v[7]);
      gput(kc + HDIM, outl[2]); gput(kc + HDIM + 64, outh[2]);
      gput(vc + HDIM, v[14]); gput(vc + HDIM + 64, v[15]);
      kv_pending = true;   // ordered before this wave's next slot publish (ar1)
    }
    // position 1: scores of heads 0, 1 against positions 0, 1
    float d[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      d[2 * h] = fmaf(outl[h], k0l, outh[h] * k0h);
      d[2 * h + 1] = fmaf(outl[h], outl[2], outh[h] * outh[2]);
    }
    group_sum_n<64>(d);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float s0 = d[2 * h] * a.scale, s1 = d[2 * h + 1] * a.scale;
      const float M = fmaxf(s0, s1);
      const float p0 = __expf(s0 - M), p1 = __expf(s1 - M);
      const float rz = rcp_f(p0 + p1);
      put_one_n(NS + wv, 128 * h + c, fmaf(p1, v[14], p0 * v[6]) * rz);
      put_one_n(NS + wv, 128 * h + c + 64, fmaf(p1, v[15], p0 * v[7]) * rz);
      put_one_n(wv, 128 * h + c, v[6]);
      put_one_n(wv, 128 * h + c + 64, v[7]);
    }
  };
  // the SwiGLU outputs of both positions (of position 1 alone after the last layer's QKV)
  auto duo_prep_down = [&](int layer, bool both, auto&& issue) SH_INLINE {
    const uint32_t o0 = ws_off(P, &ws->inter[xcd][dpar(layer, 0)][wv][0]);
    const uint32_t o1 = ws_off(P, &ws->inter[xcd][dpar(layer, 1)][wv][0]);
    if (both) {
      float v[12];
      poll_regs<6>(P, XI, tag_of(layer, T_INTER), v, [o0, o1](int i) {
        return i < XI / 2 ? o0 + 16u * (uint32_t)i : o1 + 16u * (uint32_t)(i - XI / 2);
      });
      issue();
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        put_pair_n(wv, 2 * (lane + 64 * k), v[2 * k], v[2 * k + 1]);
        put_pair_n(NS + wv, 2 * (lane + 64 * k), v[6 + 2 * k], v[7 + 2 * k]);
      }
    } else {
      float v[6];
      poll_regs<3>(P, XI / 2, tag_of(layer, T_INTER), v, [o1](int i) { return o1 + 16u * (uint32_t)i; });
      issue();
#pragma unroll
      for (int k = 0; k < 3; ++k) put_pair_n(NS + wv, 2 * (lane + 64 * k), v[2 * k], v[2 * k + 1]);
    }
  };

  // ---- attention ---------------------------------------------------------------------------
  // code predictor, wave s over stream s at length L <= 16 (f32, as the reference CP kernel):
  // lane group g takes positions j = g + 4 jj; the scores, the maximum and the sums run over
  // the 16 positions with lane-group exchanges; the output is this stream's O input.
  auto attention_cp = [&](int layer, int L) {
    const int Lold = L - 1, g = lane >> 4, d0 = 8 * (lane & 15);
    const size_t head_base = ((size_t)layer * NKVH + xcd) * (size_t)a.max_seq;
    const uint32_t bytes = (uint32_t)((size_t)NL * NKVH * (size_t)a.max_seq * HDIM * 4);
    // the cache is rewritten in this launch by another CU: L2-coherent loads (sc1); lanes
    // without a position read past the buffer end, which returns zeros
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(IO->kc, (short)0, (int)bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(IO->vc, (short)0, (int)bytes, 0x00020000);
    u32x4 kt[4][2], vt[4][2];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = g + 4 * jj;
      const bool ok = j < Lold;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const uint32_t off = ok ? (uint32_t)(((head_base + (size_t)j) * HDIM + d0 + 4 * pp) * 4) : 0xFFFFFFF0u;
        kt[jj][pp] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 16);
        vt[jj][pp] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 16);
      }
    }
    float qv[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[h][i] = s.q[wv][h][d0 + i];
    float kn8[8], vn8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { kn8[i] = s.knew[wv][d0 + i]; vn8[i] = s.vnew[wv][d0 + i]; }
    // position blocks jj (positions 4 jj .. 4 jj + 3, one per lane group) wholly past L are skipped
    // (uniform branches; their scores are -inf, their weights 0, as the masks below give them)
    float sc[8];   // [h * 4 + jj]
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = g + 4 * jj;
      float sj[2] = {0.0f, 0.0f};
      if (4 * jj < L) {
        float kv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) kv[i] = j == Lold ? kn8[i] : __uint_as_float(kt[jj][i >> 2][i & 3]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float d = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) d = fmaf(qv[h][i], kv[i], d);
          sj[h] = d;
        }
        group_sum_n<16>(sj);
      }
      sc[jj] = sj[0];
      sc[4 + jj] = sj[1];
    }
    float acc[2][8], Z[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float M = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = g + 4 * jj;
        sc[4 * h + jj] = j < L ? sc[4 * h + jj] * a.scale : -INFINITY;
        M = fmaxf(M, sc[4 * h + jj]);
      }
      M = fmaxf(M, xlane_f<4>(M));
      M = fmaxf(M, xlane_f<5>(M));
      Z[h] = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] = 0.0f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        if (4 * jj < L) {
          const int j = g + 4 * jj;
          const float p = j < L ? __expf(sc[4 * h + jj] - M) : 0.0f;
          Z[h] += p;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(p, j == Lold ? vn8[i] : __uint_as_float(vt[jj][i >> 2][i & 3]), acc[h][i]);
        }
      }
    }
    // lane groups hold different positions: sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 as
    // (a_g + a_g^1) + (a_g^2 + a_g^3), scattered: after the two exchanges lane group g holds the 4
    // values k = n + 4 ((g >> 1) & 1) + 8 (g & 1) (head k >> 3, dims d0 + (k & 7)), each summed in
    // the order a full butterfly gives (the two halves' sums commute exactly)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      Z[h] += xlane_f<4>(Z[h]);
      Z[h] += xlane_f<5>(Z[h]);
    }
    const bool hi1 = (g & 1) != 0, hi2 = (g & 2) != 0;
    float k8[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const float send = hi1 ? acc[0][m] : acc[1][m];
      const float keep = hi1 ? acc[1][m] : acc[0][m];
      k8[m] = keep + xlane_f<4>(send);
    }
    float k4[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const float send = hi2 ? k8[n] : k8[n + 4];
      const float keep = hi2 ? k8[n + 4] : k8[n];
      k4[n] = keep + xlane_f<5>(send);
    }
    const float rz = rcp_f(hi1 ? Z[1] : Z[0]);
    const int e = 128 * (hi1 ? 1 : 0) + d0 + (hi2 ? 4 : 0);
    put_pair(e, k4[0] * rz, k4[1] * rz);
    put_pair(e + 2, k4[2] * rz, k4[3] * rz);
  };
  // backbone: unit li of this XCD's KV head (stream us, positions [c0, c1)), f32 softmax. Wave w
  // takes positions c0 + APASS * pass + 32 w + 4 jj + g (lane group g, jj < AJJ) with its own
  // running maximum; the 8 waves' (m, l, acc) are merged in LDS and published unnormalised.
  // The first pass's K/V tile was issued in the QKV step; later passes load their own.
  auto load_kv = [&](TKV& t, int layer, int us, int b0, int lim) {
    const IOP io = IO0 + us;
    const bf16_t* kc = reinterpret_cast<const bf16_t*>(io->kc);
    const bf16_t* vc = reinterpret_cast<const bf16_t*>(io->vc);
    const size_t head_base = ((size_t)layer * NKVH + xcd) * (size_t)a.max_seq;
    const int g = lane >> 4, d0 = 8 * (lane & 15);
#pragma unroll
    for (int jj = 0; jj < AJJ; ++jj) {
      const int pos = b0 + 4 * AJJ * wv + 4 * jj + g;
      const bool ok = pos < lim;
      // positions past lim read slot 0 (finite cache data): their scores are masked to -inf and
      // their V weighs 0, so no select on the loaded value (it would wait for the load here)
      const size_t off = (head_base + (size_t)(ok ? pos : 0)) * HDIM + d0;
      t.k[jj] = ldw(kc + off);
      t.v[jj] = ldw(vc + off);
    }
  };
  struct Unit { int us, L, c0, c1; };
  auto unit_of = [&]() {
    Unit u;
    u.us = a.unit_stream[li];
    if (u.us >= 0 && !is_live(u.us)) u.us = -1;
    const IOP io = IO0 + (u.us >= 0 ? u.us : 0);
    u.L = io->pos + 1;
    u.c0 = u.us >= 0 ? (li - io->u0) * io->P : 0;
    u.c1 = u.us >= 0 ? min(u.L, u.c0 + io->P) : 0;
    return u;
  };
  auto load_kv_first = [&](TKV& t, int layer) {
    const Unit u = unit_of();
    load_kv(t, layer, u.us >= 0 ? u.us : 0, u.c0, u.us >= 0 ? min(u.c1, u.L - 1) : 0);
  };
  auto attention_unit = [&](int lp, int layer, TKV& t) {
    const Unit u = unit_of();
    const int g = lane >> 4, d0 = 8 * (lane & 15);
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f}, acc[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] = 0.0f;
    if (u.us >= 0) {
      const int Lold = u.L - 1;
      float qv[2][8], kn8[8], vn8[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[h][i] = s.q[u.us][h][d0 + i];
#pragma unroll
      for (int i = 0; i < 8; ++i) { kn8[i] = s.knew[u.us][d0 + i]; vn8[i] = s.vnew[u.us][d0 + i]; }
      for (int b0 = u.c0; b0 < u.c1; b0 += APASS) {
        if (b0 > u.c0) load_kv(t, layer, u.us, b0, min(u.c1, Lold));
        // blocks of 4 positions (one per lane group) wholly past the unit's end are skipped
        // (wave-uniform branches); their scores are -inf and their weights 0, as the masks give them
        const int wb0 = b0 + 4 * AJJ * wv;   // the wave's first position of this pass
        float sc[2 * AJJ];   // [h * AJJ + jj]
#pragma unroll
        for (int jj = 0; jj < AJJ; ++jj) {
          const int pos = wb0 + 4 * jj + g;
          float sj[2] = {0.0f, 0.0f};
          if (wb0 + 4 * jj < u.c1) {
            const u32x4 w = t.k[jj];
            float kv[8] = {bflo(w.x), bfhi(w.x), bflo(w.y), bfhi(w.y), bflo(w.z), bfhi(w.z), bflo(w.w), bfhi(w.w)};
#pragma unroll
            for (int i = 0; i < 8; ++i) kv[i] = pos == Lold ? kn8[i] : kv[i];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              float d = 0.0f;
#pragma unroll
              for (int i = 0; i < 8; ++i) d = fmaf(qv[h][i], kv[i], d);
              sj[h] = d;
            }
            group_sum_n<16>(sj);
          }
          sc[jj] = sj[0];
          sc[AJJ + jj] = sj[1];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float mx = -INFINITY;
#pragma unroll
          for (int jj = 0; jj < AJJ; ++jj) {
            const int pos = b0 + 4 * AJJ * wv + 4 * jj + g;
            sc[h * AJJ + jj] = pos < u.c1 ? sc[h * AJJ + jj] * a.scale : -INFINITY;
            mx = fmaxf(mx, sc[h * AJJ + jj]);
          }
          mx = fmaxf(mx, xlane_f<4>(mx));
          mx = fmaxf(mx, xlane_f<5>(mx));
          const float mn = fmaxf(m[h], mx);
          if (mn != -INFINITY) {   // wave-uniform: some position of this wave is valid
            const float alpha = m[h] == -INFINITY ? 0.0f : __expf(m[h] - mn);
            l[h] *= alpha;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[h][i] *= alpha;
#pragma unroll
            for (int jj = 0; jj < AJJ; ++jj) {
              if (wb0 + 4 * jj < u.c1) {
                const float p = sc[h * AJJ + jj] == -INFINITY ? 0.0f : __expf(sc[h * AJJ + jj] - mn);
                const int pos = wb0 + 4 * jj + g;
                const u32x4 w = t.v[jj];
                float vv[8] = {bflo(w.x), bfhi(w.x), bflo(w.y), bfhi(w.y), bflo(w.z), bfhi(w.z), bflo(w.w), bfhi(w.w)};
                l[h] += p;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(p, pos == Lold ? vn8[i] : vv[i], acc[h][i]);
              }
            }
            m[h] = mn;
          }
        }
      }
    }
    // the wave's totals over its 4 lane groups, (a_g + a_g^1) + (a_g^2 + a_g^3); the accumulators
    // scattered so that lane group g ends with head g & 1, dims d0 + 4 ((g >> 1) & 1) + n (n < 4),
    // each summed in the order a full butterfly gives (the halves' sums commute exactly)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      l[h] += xlane_f<4>(l[h]);
      l[h] += xlane_f<5>(l[h]);
      if (lane == 0) { s.wpart[wv][h][HDIM] = m[h]; s.wpart[wv][h][HDIM + 1] = l[h]; }
    }
    {
      const bool hi1 = (g & 1) != 0, hi2 = (g & 2) != 0;
      float k8[8];
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const float send = hi1 ? acc[0][n] : acc[1][n];
        const float keep = hi1 ? acc[1][n] : acc[0][n];
        k8[n] = keep + xlane_f<4>(send);
      }
      float* dst = &s.wpart[wv][hi1 ? 1 : 0][d0 + (hi2 ? 4 : 0)];
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const float send = hi2 ? k8[n] : k8[n + 4];
        const float keep = hi2 ? k8[n + 4] : k8[n];
        dst[n] = keep + xlane_f<5>(send);
      }
    }
    step_barrier();
    if (u.us >= 0 && tid < 2 * HDIM) {
      const int h = tid >> 7, d = tid & 127;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < SWAV; ++w) M = fmaxf(M, s.wpart[w][h][HDIM]);
      float As = 0.0f, Zs = 0.0f;
#pragma unroll
      for (int w = 0; w < SWAV; ++w) {
        const float mw = s.wpart[w][h][HDIM];
        const float e = mw == -INFINITY ? 0.0f : __expf(mw - M);
        As = fmaf(e, s.wpart[w][h][d], As);
        Zs = fmaf(e, s.wpart[w][h][HDIM + 1], Zs);
      }
      uint64_t* dst = &ws->attp[xcd][lp & 1][li][h][0];
      const uint32_t tg = tag_of(lp, T_ATT);
      pub_local(dst + d, As, tg);
      if (d == 0) { pub_local(dst + HDIM, M, tg); pub_local(dst + HDIM + 1, Zs, tg); }
    }
  };

  // ---- projections on MFMA ------------------------------------------------------------------
  // Weight fragments: lane l holds 8 consecutive bf16 of row (l & 15) of a 16-row block at
  // columns 32 kb + 8 (l >> 4) (the v_mfma_f32_16x16x32_bf16 A layout). Rows past the tile's
  // valid count are read from a valid row (no load under a branch, no select on the loaded
  // value, which would wait for it); their output rows are never summed or published.
  auto wld = [&](const bf16_t* p) -> u32x4 {
    if constexpr (BB) return ldw_nt(p); else return ldw(p);
  };
  auto load_q = [&](TQ& t, int layer) {
    const int i = lane & 15, kg = lane >> 4;
    const int lr = 16 * li + i;   // local row of the XCD's 512 (a workgroup's 16 rows share one block)
    const bf16_t* row;
    if (16 * li < 256) row = lw(LW, layer, W_Q) + (size_t)(256 * xcd + lr) * HID;
    else if (16 * li < 384) row = lw(LW, layer, W_K) + (size_t)(128 * xcd + lr - 256) * HID;
    else row = lw(LW, layer, W_V) + (size_t)(128 * xcd + lr - 384) * HID;
#pragma unroll
    for (int j = 0; j < 4; ++j) t.p[j] = wld(row + 32 * (4 * wv + j) + 8 * kg);
  };
  auto load_o = [&](TO& t, int layer) {
    const int i = lane & 15, kg = lane >> 4, tile = wv >> 2;
    const bf16_t* row = lw(LW, layer, W_O) + (size_t)(32 * li + 16 * tile + i) * (NQH * HDIM) + 256 * xcd;
#pragma unroll
    for (int j = 0; j < 2; ++j) t.p[j] = wld(row + 32 * (2 * (wv & 3) + j) + 8 * kg);
  };
  // the gate/up tile, issued in two halves: `part` takes K-blocks 4 part .. 4 part + 3 of the wave's 8
  auto load_g_half = [&](TG& t, int layer, int part) {
    const int i = lane & 15, kg = lane >> 4, tile = wv >> 2;
    const bf16_t* row = lw(LW, layer, tile ? W_UP : W_GATE) + (size_t)(XI * xcd + 12 * li + (i < 12 ? i : 0)) * HID;
#pragma unroll
    for (int j = 0; j < 4; ++j) t.p[4 * part + j] = wld(row + 32 * (8 * (wv & 3) + 4 * part + j) + 8 * kg);
  };
  auto load_d = [&](TD& t, int layer) {
    const int i = lane & 15, kg = lane >> 4, tile = wv >> 2;
    const bf16_t* row = lw(LW, layer, W_DOWN) + (size_t)(32 * li + 16 * tile + i) * INTER + XI * xcd;
#pragma unroll
    for (int j = 0; j < 3; ++j) t.p[j] = wld(row + 32 * (3 * (wv & 3) + j) + 8 * kg);
  };
  const int head_rows = (cp ? a.cp_vocab : a.vocab) / NWG;   // rows of this workgroup (<= 16)
  auto head_w = [&](int pi) -> const bf16_t* { return cp ? ld_const(a.cp_heads + (pi - 1)) : a.head; };
  auto load_h = [&](TQ& t, const bf16_t* W) {
    const int i = lane & 15, kg = lane >> 4;
    const bf16_t* row = W + (size_t)(wg * head_rows + (i < head_rows ? i : 0)) * HID;
#pragma unroll
    for (int j = 0; j < 4; ++j) t.p[j] = wld(row + 32 * (4 * wv + j) + 8 * kg);
  };
  // The wave's K-blocks kb0 .. kb0 + NB - 1 of its tile against the 16 input columns (hi and mid
  // pieces of the 8 streams) and the 8 lo columns; the partial of (row, stream) goes to
  // red[wave][row][stream] = (hi + mid) + lo. Output layout: lane l holds rows 4 (l >> 4) + e
  // of column l & 15.
  auto gemv = [&](const auto& tp, int kb0) {
    constexpr int NB = sizeof(tp) / sizeof(u32x4);
    const int n = lane & 15, kg = lane >> 4;
    f32x4 c1 = {0.0f, 0.0f, 0.0f, 0.0f}, c2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = 32 * (kb0 + j) + 8 * kg;
      const u32x4 b1 = *reinterpret_cast<const u32x4*>(&s.xb[(n >> 3) * XPS + (n & 7) * KP + k]);
      const u32x4 b2 = *reinterpret_cast<const u32x4*>(&s.xb[2 * XPS + (n & 7) * KP + k]);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(tp[j]), as_bf8(b1), c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(tp[j]), as_bf8(b2), c2, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = (c1[e] + ror8(c1[e])) + c2[e];
      if (n < 8) s.red[wv][4 * kg + e][n] = v;
    }
  };
  // The same over all 16 input columns (the two-column pass): one MFMA per piece, and the partial
  // of (row, column n) is (hi + mid) + lo, as above.
  auto gemv2 = [&](const auto& tp, int kb0) {
    constexpr int NB = sizeof(tp) / sizeof(u32x4);
    const int n = lane & 15, kg = lane >> 4;
    f32x4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = {0.0f, 0.0f, 0.0f, 0.0f}, c2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = 32 * (kb0 + j) + 8 * kg;
      const u32x4 b0 = *reinterpret_cast<const u32x4*>(&s.xb[n * KP + k]);
      const u32x4 b1 = *reinterpret_cast<const u32x4*>(&s.xb[XPS + n * KP + k]);
      const u32x4 b2 = *reinterpret_cast<const u32x4*>(&s.xb[2 * XPS + n * KP + k]);
      c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(tp[j]), as_bf8(b0), c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(tp[j]), as_bf8(b1), c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(tp[j]), as_bf8(b2), c2, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) s.red[wv][4 * kg + e][n] = (c0[e] + c1[e]) + c2[e];
  };
  // sum of the partials of waves w0 .. w0 + nw - 1 (fixed order)
  auto red_sum = [&](int w0, int nw, int r, int st) {
    float v = 0.0f;
    for (int w = 0; w < nw; ++w) v += s.red[w0 + w][r][st];
    return v;
  };

  // ---- selection ----------------------------------------------------------------------------
  // greedy code-predictor head of this wave's stream: two-level exchange of the workgroup bests
  // (value, lowest id on ties): the 32 of this XCD through L2, then the 8 XCD bests read from the
  // copies of workgroup index li
  auto select_greedy = [&](int pi) -> int {
    const uint32_t tg = a.tag_base + TAG_HEAD + (uint32_t)pi;
    const int par = pi & 1;
    float cv[2];
    {
      const uint32_t o = ws_off(P, &ws->hloc[xcd][par][wv][0]);
      poll_regs<1>(P, WPX, tg, cv, [o](int i) { return o + 16u * (uint32_t)i; });
    }
    float bv = lane < WPX ? cv[0] : -INFINITY;
    int bi = lane < WPX ? (int)__float_as_uint(cv[1]) : 0x7fffffff;
    best_merge(bv, bi, xlane_f<0>(bv), (int)xlane<0>((uint32_t)bi));
    best_merge(bv, bi, xlane_f<1>(bv), (int)xlane<1>((uint32_t)bi));
    best_merge(bv, bi, xlane_f<2>(bv), (int)xlane<2>((uint32_t)bi));
    best_merge(bv, bi, xlane_f<3>(bv), (int)xlane<3>((uint32_t)bi));
    best_merge(bv, bi, xlane_f<4>(bv), (int)xlane<4>((uint32_t)bi));
    if (lane == 0) {
      const u32x4 d = {__float_as_uint(bv), tg, (uint32_t)bi, tg};
      __builtin_amdgcn_raw_buffer_store_b128(d, P.rs, (int)ws_off(P, &ws->hx[par][wv][li][2 * xcd]), 0, 16);
    }
    {
      const uint32_t o = ws_off(P, &ws->hx[par][wv][li][0]);
      poll_regs<1>(P, NXCD, tg, cv, [o](int i) { return o + 16u * (uint32_t)i; });
    }
    bv = lane < NXCD ? cv[0] : -INFINITY;
    bi = lane < NXCD ? (int)__float_as_uint(cv[1]) : 0x7fffffff;
    best_merge(bv, bi, xlane_f<0>(bv), (int)xlane<0>((uint32_t)bi));
    best_merge(bv, bi, xlane_f<1>(bv), (int)xlane<1>((uint32_t)bi));
    best_merge(bv, bi, xlane_f<2>(bv), (int)xlane<2>((uint32_t)bi));
    bi = __builtin_amdgcn_readfirstlane(bi);
    return (bi >= 0 && bi < a.cp_vocab) ? bi : 0;   // a timed-out poll may leave garbage
  };
  // the stream's whole logit vector into LDS, then mask, penalty and wave_select (its own
  // workgroup only: the selection scratch overlays the projection inputs)
  auto select_full = [&](int pi) -> int {
    const int n = cp ? a.cp_vocab : a.vocab;
    poll_vec_long(P, &ws->logits[pi & 1][wv][0], n, a.tag_base + TAG_HEAD + (uint32_t)pi, s.z.stage);
    SelParams sp = a.sel;
    sp.seed = IO->seed;
    if (cp) {
      sp.group = pi;   // CP head pi-1 selects codebook group pi
    } else {
      // suppress ids [V-1024, V) except EOS (generator.py:71-75)
      if (a.mask_tail)
        for (int i = lane; i < n; i += 64)
          if (i >= n - 1024 && i != a.eos_id) s.z.stage[i] = -INFINITY;
      // repetition penalty, once per distinct id, bf16 arithmetic (generator.py:161-167)
      if (a.rep_penalty != 1.0f && IO->n_history > 0) {
        for (int i = lane; i < MAXV / 32; i += 64) s.pen_bits[wv][i] = 0u;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        for (int i = lane; i < IO->n_history; i += 64) {
          const int id = IO->history[i];
          if (id >= 0 && id < n) atomicOr(&s.pen_bits[wv][id >> 5], 1u << (id & 31));
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        for (int i = lane; i < n; i += 64) {
          if (s.pen_bits[wv][i >> 5] & (1u << (i & 31))) {
            const float v = s.z.stage[i];
            s.z.stage[i] = rbf(v > 0.f ? v / a.rep_penalty : v * a.rep_penalty);
          }
        }
      }
      if (a.suppress_eos && a.eos_id >= 0 && a.eos_id < n && lane == 0) s.z.stage[a.eos_id] = -INFINITY;
      sp.group = 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return sh_wave_select(s.z.stage, n, sp, &s.z.sel);
  };

  // =========================================================================================
  // Step schedule: every wave runs the same steps and barriers. A projection step is
  //   barrier (inputs in LDS) -> MFMA over the tile -> next tile issued -> barrier (partials in
  //   LDS) -> sums published -> each wave's vector work for its stream (its next inputs).
  // =========================================================================================
  TQ tq;
  TO to;
  TG tgu;
  TD td;
  TKV tkv;
  load_q(tq, 0);
  // the code-predictor frame runs positions 0 and 1 as one two-column pass, then position 1's head
  const bool duo = cp && a.n_pos >= 2;
  int npass = 0;   // layer passes begun: the first one's waits run under the entry cap
  auto pass_begin = [&]() {
    if (npass == 1) P.ec.spin_cap = a.spin_cap;
    ++npass;
  };
  if (me) {
    prep_input0(0, wv, s.xres[wv]);
    if (duo) prep_input0(1, NS + wv, s.xres1[wv]);
  }
  for (int pi = duo ? 1 : 0; pi < a.n_pos; ++pi) {
    const int pos = BB ? IO->pos : pi;
    const bool last_pos = pi == a.n_pos - 1;
    const bool head = has_head(pi);
    if constexpr (!BB) {
      if (duo && pi == 1) {
        for (int layer = 0; layer < NL; ++layer) {
          lane = opaque(lane);
          tid = opaque(tid);
          const bool last_layer = layer == NL - 1;
          pass_begin();
          // ---- QKV, both positions
          step_barrier();
          stamp(0);
          gemv2(tq.p, 4 * wv);
          step_barrier();
          stamp(1);
          if (tid < 16 * 2 * NS) {
            const int n = tid >> 4, st = n & (NS - 1), c = n / NS, r = tid & 15;
            const float v = red_sum(0, SWAV, r, n);
            const int lr = 16 * li + r, cc = lr & 127;
            if (is_live(st))
              pub_local(&ws->qkv[xcd][dpar(layer, c)][st][(lr & ~127) + 2 * (cc & 63) + (cc >> 6)], v, tag_of(layer, T_QKV));
          }
          stamp(14);
          {
            auto iss = [&]() SH_INLINE { load_o(to, layer); };
            if (me) duo_prep_att(layer, iss);
            else iss();
          }
          stamp(2 + wv);
          ++nstep;
          // ---- O projection (position 0's stops after its last QKV)
          step_barrier();
          stamp(0);
          gemv2(to.p, 2 * (wv & 3));
          step_barrier();
          stamp(1);
          {
            const int n = tid >> 5, st = n & (NS - 1), c = n / NS, tile = (tid >> 4) & 1, r = tid & 15;
            const float v = red_sum(4 * tile, 4, r, n);
            if (is_live(st) && (c == 1 || !last_layer))
              pub_cross(&ws->opart[dpar(layer, c)][xcd][st][32 * li + 16 * tile + r], v, tag_of(layer, T_OPART));
          }
          stamp(14);
          {
            // the gate/up tile in two halves, as in the single-column pass (launch 1,460 -> 1,455 us)
            auto iss = [&]() SH_INLINE { load_g_half(tgu, layer, 0); };
            auto iss2 = [&]() SH_INLINE { load_g_half(tgu, layer, 1); };
            if (me) {
              // both columns' sums published before either gather
              if (!last_layer) ar1(layer, dpar(layer, 0), s.xres[wv]);
              ar1(layer, dpar(layer, 1), s.xres1[wv]);
              if (!last_layer)
                cp_prep_vec(&ws->h1[xcd][dpar(layer, 0)][wv][0], tag_of(layer, T_H1), lw(LW, layer, W_LNPOST), s.h1res[wv],
                            wv, []() SH_INLINE {});
              cp_prep_vec2(&ws->h1[xcd][dpar(layer, 1)][wv][0], tag_of(layer, T_H1), lw(LW, layer, W_LNPOST), s.h1res1[wv],
                           NS + wv, iss, iss2);
            } else {
              iss();
              iss2();
            }
          }
          stamp(2 + wv);
          ++nstep;
          // ---- gate / up + SiLU
          step_barrier();
          stamp(0);
          gemv2(tgu.p, 8 * (wv & 3));
          step_barrier();
          stamp(1);
          if (tid < 12 * 2 * NS) {
            const int n = tid / 12, st = n & (NS - 1), c = n / NS, r = tid - 12 * n;
            const float gt = red_sum(0, 4, r, n), up = red_sum(4, 4, r, n);
            const float act = gt / (1.0f + __expf(-gt)) * up;
            if (is_live(st) && (c == 1 || !last_layer))
              pub_local(&ws->inter[xcd][dpar(layer, c)][st][12 * li + r], act, tag_of(layer, T_INTER));
          }
          stamp(14);
          {
            auto iss = [&]() SH_INLINE { load_d(td, layer); };
            if (me) duo_prep_down(layer, !last_layer, iss);
            else iss();
          }
          stamp(2 + wv);
          ++nstep;
          // ---- down projection
          step_barrier();
          stamp(0);
          gemv2(td.p, 3 * (wv & 3));
          step_barrier();
          stamp(1);
          {
            const int n = tid >> 5, st = n & (NS - 1), c = n / NS, tile = (tid >> 4) & 1, r = tid & 15;
            const float v = red_sum(4 * tile, 4, r, n);
            if (is_live(st) && (c == 1 || !last_layer))
              pub_cross(&ws->dpart[dpar(layer, c)][xcd][st][32 * li + 16 * tile + r], v, tag_of(layer, T_DPART));
          }
          stamp(14);
          {
            // next: both positions' next-layer inputs, or position 1's final norm (the head's input)
            auto iss = [&]() SH_INLINE {
              if (!last_layer) load_q(tq, layer + 1);
              else load_h(tq, head_w(1));
            };
            if (me) {
              if (!last_layer) {
                ar2(layer, dpar(layer, 0), s.h1res[wv]);
                ar2(layer, dpar(layer, 1), s.h1res1[wv]);
                cp_prep_vec(&ws->xl[xcd][dpar(layer, 0)][wv][0], tag_of(layer, T_XL), lw(LW, layer + 1, W_LNIN), s.xres[wv],
                            wv, []() SH_INLINE {});
                cp_prep_vec(&ws->xl[xcd][dpar(layer, 1)][wv][0], tag_of(layer, T_XL), lw(LW, layer + 1, W_LNIN),
                            s.xres1[wv], NS + wv, iss);
              } else {
                ar2(layer, dpar(layer, 1), s.h1res1[wv]);
                cp_prep_final(layer, dpar(layer, 1), iss);
              }
            } else {
              iss();
            }
          }
          stamp(2 + wv);
          ++nstep;
        }
      }
    }
    for (int layer = 0; layer < ((!BB && duo && pi == 1) ? 0 : NL); ++layer) {
      lane = opaque(lane);
      tid = opaque(tid);
      const int lp = pi * NL + layer;
      const int par = lp & 1;
      const bool last_layer = layer == NL - 1;
      pass_begin();
      // ---- QKV
      step_barrier();
      stamp(0);
      gemv(tq.p, 4 * wv);
      step_barrier();
      stamp(1);
      if (tid < 16 * NS) {
        const int st = tid >> 4, r = tid & 15;
        const float v = red_sum(0, SWAV, r, st);
        // slot order pairs the rotate_half partners: channel c' of head block h goes to slot
        // 128 h + 2 (c' mod 64) + c' / 64, so one 16-byte pair holds channels c and c + 64
        const int lr = 16 * li + r, cc = lr & 127;
        if (is_live(st)) pub_local(&ws->qkv[xcd][par][st][(lr & ~127) + 2 * (cc & 63) + (cc >> 6)], v, tag_of(lp, T_QKV));
      }
      stamp(14);
      // the next tiles go out after the publish: a wave's vector-memory results return in issue
      // order, so a poll issued behind a tile load would wait for the tile
      if constexpr (BB) {
        auto iss = [&]() SH_INLINE { load_kv_first(tkv, layer); load_o(to, layer); };
        if (me) prep_att(lp, layer, pos, iss);
        else iss();
      } else {
        // (position 0 of a frame of two or more positions runs in the two-column pass above)
        auto iss = [&]() SH_INLINE { load_o(to, layer); };
        if (me) cp_prep_att(lp, layer, pos, iss);
        else iss();
      }
      stamp(2 + wv);
      ++nstep;
      // ---- attention (backbone: its own step; code predictor: local, before the O projection)
      if constexpr (BB) {
        step_barrier();
        stamp(0);
        attention_unit(lp, layer, tkv);
        stamp(1);
        if (me) prep_o(lp);
        stamp(2 + wv);
        ++nstep;
      } else {
        if (me) attention_cp(layer, pi + 1);
        stamp(13);
      }
      // ---- O projection (cross-XCD partials)
      step_barrier();
      stamp(0);
      gemv(to.p, 2 * (wv & 3));
      step_barrier();
      stamp(1);
      if (tid < 32 * NS) {
        const int st = tid >> 5, tile = (tid >> 4) & 1, r = tid & 15;
        const float v = red_sum(4 * tile, 4, r, st);
        if (is_live(st)) pub_cross(&ws->opart[par][xcd][st][32 * li + 16 * tile + r], v, tag_of(lp, T_OPART));
      }
      stamp(14);
      {
        // the gate/up tile (48 KB per workgroup) in two halves, the second after the vector work:
        // issued whole, its burst lands on the other workgroups' gathers (config 4: code-predictor
        // launch 1,488 -> 1,459 us, backbone 858 -> 849 us; a 2 + 6 split gained nothing, 6 + 2 less)
        auto iss = [&]() SH_INLINE { stamp(12); load_g_half(tgu, layer, 0); };
        auto iss2 = [&]() SH_INLINE { load_g_half(tgu, layer, 1); };
        if (me) {
          ar1(lp, par, s.xres[wv]);
          stamp(11);
          cp_prep_vec2(&ws->h1[xcd][par][wv][0], tag_of(lp, T_H1), lw(LW, layer, W_LNPOST), s.h1res[wv], wv, iss, iss2);
        } else {
          iss();
          iss2();
        }
      }
      stamp(2 + wv);
      ++nstep;
      // ---- gate / up + SiLU
      step_barrier();
      stamp(0);
      gemv(tgu.p, 8 * (wv & 3));
      step_barrier();
      stamp(1);
      if (tid < 12 * NS) {
        const int st = tid / 12, r = tid - 12 * st;
        const float gt = red_sum(0, 4, r, st), up = red_sum(4, 4, r, st);
        const float act = gt / (1.0f + __expf(-gt)) * up;
        if (is_live(st)) pub_local(&ws->inter[xcd][par][st][12 * li + r], act, tag_of(lp, T_INTER));
      }
      stamp(14);
      {
        auto iss = [&]() SH_INLINE { load_d(td, layer); };
        if (me) cp_prep_down(lp, iss);
        else iss();
      }
      stamp(2 + wv);
      ++nstep;
      // ---- down projection (cross-XCD partials)
      step_barrier();
      stamp(0);
      gemv(td.p, 3 * (wv & 3));
      step_barrier();
      stamp(1);
      if (tid < 32 * NS) {
        const int st = tid >> 5, tile = (tid >> 4) & 1, r = tid & 15;
        const float v = red_sum(4 * tile, 4, r, st);
        if (is_live(st)) pub_cross(&ws->dpart[par][xcd][st][32 * li + 16 * tile + r], v, tag_of(lp, T_DPART));
      }
      stamp(14);
      if constexpr (BB) {
        if (!last_layer) {
          // the next layer's QKV tile goes out after the gather's last poll
          auto iss = [&]() SH_INLINE { load_q(tq, layer + 1); };
          if (me) {
            ar2(lp, par, s.h1res[wv]);
            cp_prep_vec(&ws->xl[xcd][par][wv][0], tag_of(lp, T_XL), lw(LW, layer + 1, W_LNIN), s.xres[wv], wv, iss);
          } else {
            iss();
          }
        } else {
          if (head) load_h(tq, head_w(pi));
          else if (!last_pos) load_q(tq, 0);
          if (me) {
            if (head || last_pos) { ar2(lp, par, s.h1res[wv]); prep_final(lp); }
            else prep_input0(pi + 1, wv, s.xres[wv]);
          }
        }
      } else {
        // next: the following layer's input, the final norm (a head follows every position
        // from 1 on), or, after position 0 (whose output feeds no head), position 1's input
        auto iss = [&]() SH_INLINE {
          if (!last_layer) load_q(tq, layer + 1);
          else if (head) load_h(tq, head_w(pi));
          else if (!last_pos) load_q(tq, 0);
        };
        if (me) {
          if (!last_layer) {
            ar2(lp, par, s.h1res[wv]);
            cp_prep_vec(&ws->xl[xcd][par][wv][0], tag_of(lp, T_XL), lw(LW, layer + 1, W_LNIN), s.xres[wv], wv, iss);
          } else if (head || last_pos) {
            ar2(lp, par, s.h1res[wv]);
            cp_prep_final(lp, par, iss);
          } else {
            cp_prep_input0(pi + 1, iss);
          }
        } else {
          iss();
        }
      }
      stamp(2 + wv);
      ++nstep;
    }
    if (head) {
      lane = opaque(lane);
      tid = opaque(tid);
      step_barrier();
      stamp(0);
      gemv(tq.p, 4 * wv);
      step_barrier();
      stamp(1);
      const uint32_t tg = a.tag_base + TAG_HEAD + (uint32_t)pi;
      const int row0 = wg * head_rows;
      if (tid < 16 * NS) {
        // logits are bf16 values, as the reference's torch.mv over bf16 operands returns them
        // (generator.py:158, :351); ties go to the lowest id, as torch.argmax
        const int st = tid >> 4, r = tid & 15;
        const float lv = rbf(red_sum(0, SWAV, r, st));
        const bool ok = r < head_rows && is_live(st);
        if (cp_greedy) {
          float bv = ok ? lv : -INFINITY;
          int bi = row0 + r;
          best_merge(bv, bi, xlane_f<0>(bv), (int)xlane<0>((uint32_t)bi));
          best_merge(bv, bi, xlane_f<1>(bv), (int)xlane<1>((uint32_t)bi));
          best_merge(bv, bi, xlane_f<2>(bv), (int)xlane<2>((uint32_t)bi));
          best_merge(bv, bi, xlane_f<3>(bv), (int)xlane<3>((uint32_t)bi));
          if (r == 0 && is_live(st)) {
            const u32x4 d = {__float_as_uint(bv), tg, (uint32_t)bi, tg};
            __builtin_amdgcn_raw_buffer_store_b128(d, P.rs, (int)ws_off(P, &ws->hloc[xcd][pi & 1][st][2 * li]), 0, 0);
          }
        } else if (ok) {
          pub_cross(&ws->logits[pi & 1][st][row0 + r], lv, tg);
          if (!cp && (IO0 + st)->out_logits) (IO0 + st)->out_logits[row0 + r] = lv;
        }
      }
      stamp(14);
      if constexpr (BB) {
        if (!last_pos) load_q(tq, 0);
      }
      if (cp) {
        int tok = 0;
        if (cp_greedy) {
          if (me) tok = select_greedy(pi);
        } else {
          // sampled: the stream's own workgroup selects and publishes the id; every workgroup
          // reads it after the barrier that ends the selection scratch's use of the inputs
          if (me && wg == wv) {
            const int t = select_full(pi);
            if (lane == 0) {
              const u32x4 d = {(uint32_t)t, tg, (uint32_t)t, tg};
              __builtin_amdgcn_raw_buffer_store_b128(d, P.rs, (int)ws_off(P, &ws->tok[pi & 1][wv][0]), 0, 16);
            }
          }
          step_barrier();
          if (me) {
            float cv[2];
            const uint32_t o = ws_off(P, &ws->tok[pi & 1][wv][0]);
            [[clang::always_inline]] poll_regs<1>(P, 1, tg, cv, [o](int) { return o; });
            const int t = __builtin_amdgcn_readfirstlane((int)__float_as_uint(cv[0]));
            tok = (t >= 0 && t < a.cp_vocab) ? t : 0;
          }
        }
        if (me) {
          if (lane == 0) s.tok[wv][pi - 1] = tok;
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          if constexpr (BB) {
            if (!last_pos) prep_input0(pi + 1, wv, s.xres[wv]);
          }
        }
        if constexpr (!BB) {
          auto iss = [&]() SH_INLINE { if (!last_pos) load_q(tq, 0); };
          if (me && !last_pos) cp_prep_input0(pi + 1, iss);
          else iss();
        }
      } else if (me && wg == wv) {
        const int t = select_full(pi);
        if (lane == 0 && IO->out_token) *IO->out_token = t;
      }
      stamp(2 + wv);
      ++nstep;
    }
  }

  // ---- code-predictor frame epilogue (the stream's own workgroup): ids and the bf16 combine
  if (cp && me && wg == wv) {
    if (lane == 0) {
      IO->out_tokens[0] = *IO->g0;
      for (int g = 0; g < a.n_groups; ++g) IO->out_tokens[1 + g] = s.tok[wv][g];
    }
    // s.comb holds emb_bb[g0] + emb_0[t_0] + ... + emb_{n-2}[t_{n-2}]; the last group's row and
    // the text row complete it (generator.py:356-362)
    const int gl = a.n_groups - 1;
    const auto* lr = gmem(reinterpret_cast<const uint32_t*>(s.embp[gl] + (size_t)s.tok[wv][gl] * HID));
    uint32_t wl[8], wt[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) wl[k] = lr[lane + 64 * k];
    if (IO->text_row) {
      const auto* tr = gmem(reinterpret_cast<const uint32_t*>(IO->text_row));
#pragma unroll
      for (int k = 0; k < 8; ++k) wt[k] = tr[lane + 64 * k];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = 2 * (lane + 64 * k);
      float a0 = rbf(s.comb[e] + bflo(wl[k])), a1 = rbf(s.comb[e + 1] + bfhi(wl[k]));
      if (IO->text_row) { a0 = rbf(a0 + bflo(wt[k])); a1 = rbf(a1 + bfhi(wt[k])); }
      gput(reinterpret_cast<uint32_t*>(IO->out_combined) + (e >> 1), (uint32_t)f2bf(a0) | ((uint32_t)f2bf(a1) << 16));
    }
  }
}

template __global__ void qtts_shared_kernel<true>(const SArgs a);
template __global__ void qtts_shared_kernel<false>(const SArgs a);

}  // namespace sh
}  // namespace qtts

// =========================================================================================
// Host side
// =========================================================================================
namespace {

// optional step timeline buffer of the weight-shared kernels; set from any host thread, read
// once per launch
std::atomic<uint64_t*> g_strace{nullptr};

using qtts::sh::SArgs;
using qtts::sh::SStream;
using qtts::sh::SWorkspace;

void base_sargs(SArgs& a, void* ws, int n_streams, const TTSLayerWeights* layers, int num_layers, const void* final_norm,
                const void* cos_t, const void* sin_t, int max_seq) {
  std::memset(&a, 0, sizeof(a));
  a.ws = reinterpret_cast<SWorkspace*>(ws);
  a.layers = layers;
  a.num_layers = num_layers;
  a.final_norm = reinterpret_cast<const qtts::bf16_t*>(final_norm);
  a.cos_t = reinterpret_cast<const qtts::bf16_t*>(cos_t);
  a.sin_t = reinterpret_cast<const qtts::bf16_t*>(sin_t);
  a.max_seq = max_seq;
  a.scale = 0.08838834764831845f;
  a.n_pos = 1;
  a.n_streams = n_streams;
  a.eos_id = -1;
  a.sel.temperature = 1.0f;
  a.sel.top_p = 1.0f;
  a.spin_cap = qtts_host::kSpinCap;
  a.entry_spin_cap = qtts_host::entry_spin_cap();
  a.trace = g_strace.load(std::memory_order_acquire);
  for (int u = 0; u < qtts::sh::NUNIT; ++u) a.unit_stream[u] = -1;
}

bool common_ok(const SArgs& a, void* ws) {
  return ws != nullptr && (reinterpret_cast<uintptr_t>(ws) & 255u) == 0 && a.layers != nullptr && a.num_layers >= 1 &&
         a.final_norm != nullptr && a.cos_t != nullptr && a.sin_t != nullptr && a.max_seq >= 1 &&
         a.num_layers * a.n_pos <= qtts::sh::MAX_LAYER_PASSES;
}

// Attention units of the backbone: each stream gets chunks in proportion to its length
// (1 .. 8, 32 in total), unit u of every KV head on workgroup u of the XCD.
void assign_units(SArgs& a) {
  const int n = a.n_streams;
  int L[qtts::sh::NS], C[qtts::sh::NS];
  long total = 0;
  for (int t = 0; t < n; ++t) { L[t] = a.io[t].pos + 1; total += L[t]; }
  int sum = 0;
  for (int t = 0; t < n; ++t) {
    int c = (int)((2L * qtts::sh::NUNIT * L[t] + total) / (2L * total));   // round(32 L / total)
    c = c < 1 ? 1 : (c > qtts::sh::UMAX ? qtts::sh::UMAX : c);
    if (c > L[t]) c = L[t];
    C[t] = c;
    sum += c;
  }
  while (sum > qtts::sh::NUNIT) {   // take a chunk from the stream with the most
    int best = 0;
    for (int t = 1; t < n; ++t) if (C[t] > C[best]) best = t;
    --C[best];
    --sum;
  }
  int u = 0;
  for (int t = 0; t < n; ++t) {
    const int P = (L[t] + C[t] - 1) / C[t];
    const int c = (L[t] + P - 1) / P;
    a.io[t].u0 = u;
    a.io[t].nu = c;
    a.io[t].P = P;
    for (int i = 0; i < c; ++i) a.unit_stream[u + i] = t;
    u += c;
  }
}

}  // namespace

extern "C" {

size_t qtts_shared_workspace_bytes(void) { return sizeof(SWorkspace); }

hipError_t qtts_debug_trace_shared(void* device_buffer, size_t bytes) {
  if (device_buffer != nullptr &&
      bytes < (size_t)qtts::NWG * qtts::sh::TRACE_STEPS * qtts::sh::TRACE_SLOTS * sizeof(uint64_t))
    return hipErrorInvalidValue;
  g_strace.store(reinterpret_cast<uint64_t*>(device_buffer), std::memory_order_release);
  return hipSuccess;
}

hipError_t qtts_shared_workspace_check(void* workspace, unsigned int* error_code, hipStream_t stream) {
  if (workspace == nullptr || error_code == nullptr) return hipErrorInvalidValue;
  SWorkspace* ws = reinterpret_cast<SWorkspace*>(workspace);
  hipError_t e = hipMemcpyAsync(error_code, &ws->err, sizeof(unsigned int), hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return e;
  if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
  if (*error_code != 0u) {
    unsigned int zero = 0u;
    e = hipMemcpy(&ws->err, &zero, sizeof(zero), hipMemcpyHostToDevice);
  }
  return e;
}

hipError_t qtts_backbone_step_shared(int n_streams, void* workspace, const TTSLayerWeights* layer_weights, int num_layers,
                                     const void* final_norm_weight, const void* cos_table, const void* sin_table,
                                     int max_seq_len, const QttsBackboneStream* streams, const void* codec_head, int vocab,
                                     int mask_tail, float repetition_penalty, int eos_id, int suppress_eos,
                                     const QttsSampling* sampling, int frame_step, hipStream_t stream) {
  if (n_streams < 1 || n_streams > qtts::sh::NS || streams == nullptr) return hipErrorInvalidValue;
  if (codec_head != nullptr && (vocab <= 0 || vocab > qtts::MAXV || vocab % qtts::NWG != 0 || vocab / qtts::NWG > 16))
    return hipErrorInvalidValue;
  SArgs a;
  base_sargs(a, workspace, n_streams, layer_weights, num_layers, final_norm_weight, cos_table, sin_table, max_seq_len);
  if (!common_ok(a, workspace)) return hipErrorInvalidValue;
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
    SStream& io = a.io[st];
    io.kc = in.k_cache;
    io.vc = in.v_cache;
    io.pos = in.position;
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
  assign_units(a);
  return qtts_host::launch_persistent((const void*)qtts::sh::qtts_shared_kernel<true>, qtts::sh::STHR, &a, &a.tag_base,
                                      workspace, 1, sizeof(SWorkspace), stream);
}

hipError_t qtts_cp_frame_shared(int n_streams, void* workspace, const CPLayerWeights* layer_weights, int num_layers,
                                const void* final_norm_weight, const void* cos_table, const void* sin_table,
                                void* k_caches, void* v_caches, int max_seq_len, const float* bb_hidden, const int* g0,
                                const void* bb_embedding, const void* const* lm_heads, const void* const* cp_embeddings,
                                int n_groups, int cp_vocab, const void* text_rows, int* out_tokens, void* out_combined,
                                int eos_id, int* done, const QttsSampling* sampling, int frame_step, hipStream_t stream) {
  if (n_streams < 1 || n_streams > qtts::sh::NS) return hipErrorInvalidValue;
  if (k_caches == nullptr || v_caches == nullptr || bb_hidden == nullptr || g0 == nullptr || bb_embedding == nullptr ||
      lm_heads == nullptr || cp_embeddings == nullptr || out_tokens == nullptr || out_combined == nullptr || done == nullptr)
    return hipErrorInvalidValue;
  // every position of the frame in one local attention pass
  if (n_groups < 1 || n_groups + 1 > qtts::sh::CP_SUB || n_groups + 1 > max_seq_len) return hipErrorInvalidValue;
  if (cp_vocab <= 0 || cp_vocab > qtts::MAXV || cp_vocab % qtts::NWG != 0 || cp_vocab / qtts::NWG > 16)
    return hipErrorInvalidValue;
  SArgs a;
  base_sargs(a, workspace, n_streams, layer_weights, num_layers, final_norm_weight, cos_table, sin_table, max_seq_len);
  a.n_pos = n_groups + 1;
  if (!common_ok(a, workspace)) return hipErrorInvalidValue;
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
    SStream& io = a.io[st];
    io.kc = reinterpret_cast<float*>(k_caches) + kv * st;
    io.vc = reinterpret_cast<float*>(v_caches) + kv * st;
    io.bb_hidden = bb_hidden + (size_t)qtts::HID * st;
    io.g0 = g0 + st;
    io.text_row = text_rows ? reinterpret_cast<const qtts::bf16_t*>(text_rows) + (size_t)qtts::HID * st : nullptr;
    io.out_tokens = out_tokens + (size_t)(n_groups + 1) * st;
    io.out_combined = reinterpret_cast<qtts::bf16_t*>(out_combined) + (size_t)qtts::HID * st;
    io.done = done + st;
    io.seed = sampling ? sampling->seed + (uint64_t)st : 0;
  }
  return qtts_host::launch_persistent((const void*)qtts::sh::qtts_shared_kernel<false>, qtts::sh::STHR, &a, &a.tag_base,
                                      workspace, 1, sizeof(SWorkspace), stream);
}

}  // extern "C"
