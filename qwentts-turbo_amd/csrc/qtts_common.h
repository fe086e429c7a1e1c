// Device-side building blocks shared by the decode kernels (gfx950 / CDNA4, wave64).
//
// Terminology:
//   XCD      one of the 8 accelerator dies of MI355X; each has 32 CUs and its own L2.
//   slot     an 8-byte exchange word {f32 value, u32 tag}. A producer publishes a value by
//            storing the word; a consumer polls the word until the tag equals the tag of the
//            current exchange. The tag travels with the value, so no fence or counter is
//            needed and a stale word can never be mistaken for a fresh one.
//   local    exchange between workgroups of one XCD: plain stores land in that XCD's L2 and
//            sc1 loads read them there (~0.5 us round).
//   cross    exchange between XCDs: sc1 stores write through to memory and sc1 loads re-read
//            it (~1.5 us round).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

namespace qtts {

constexpr int HID = 1024;         // hidden size
constexpr int INTER = 3072;       // SwiGLU intermediate size
constexpr int NQH = 16;           // query heads
constexpr int NKVH = 8;           // key/value heads
constexpr int HDIM = 128;         // head dim
constexpr int NXCD = 8;           // XCDs, one KV head each
constexpr int WPX = 32;           // workgroups per XCD
constexpr int NWG = NXCD * WPX;   // grid size (one workgroup per CU)
constexpr int NMATH = 4;          // math waves per workgroup
constexpr int NTHR = 64 * (NMATH + 1);  // + 1 poller wave
constexpr int LROWS = 512;        // q(256) + k(128) + v(128) rows owned by one XCD
constexpr int XI = INTER / NXCD;  // 384 intermediate rows per XCD
constexpr int MAXC = 16;          // max attention chunks per KV head (2 MAXC units: every workgroup of an XCD)
constexpr int APH = 130;          // attention partial of one (chunk, head): acc[128], m, l
constexpr int APS = 2 * APH;      // partial storage per chunk (both heads)
constexpr int SUBP = 64;          // positions per prefetched attention sub-block
constexpr int MAXV = 3072;        // max vocabulary of a selection head

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_t;

// ---------------------------------------------------------------------------------------
// bf16 helpers (round-to-nearest-even, as torch's f32 -> bf16 cast)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bflo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bfhi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float((uint32_t)b << 16); }
// (branch-free: a select instead of an early return, which compiled to exec-mask branching)
__device__ __forceinline__ bf16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;   // NaN: quieted, payload kept
  return (bf16_t)((u & 0x7fffffffu) > 0x7f800000u ? qnan : rne);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
// two values packed as one bf16 pair (lo in bits 0..15) with gfx950's conversion instruction
// (v_cvt_pk_bf16_f32, round to nearest even as f2bf, one VALU op for both)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// 8 bf16 weights (one 16-byte piece) dot 8 activations, accumulated in f64 (each product is
// exact in f64; only the accumulation rounds, at ~1e-16 relative).
__device__ __forceinline__ double dot8d(const u32x4 w, const double* x, double acc) {
  acc = fma((double)bflo(w.x), x[0], acc);
  acc = fma((double)bfhi(w.x), x[1], acc);
  acc = fma((double)bflo(w.y), x[2], acc);
  acc = fma((double)bfhi(w.y), x[3], acc);
  acc = fma((double)bflo(w.z), x[4], acc);
  acc = fma((double)bfhi(w.z), x[5], acc);
  acc = fma((double)bflo(w.w), x[6], acc);
  acc = fma((double)bfhi(w.w), x[7], acc);
  return acc;
}

// The same in f32 (per-lane FMA chain; the code-predictor kernel's arithmetic, as the reference's
// CP kernel accumulates in f32).
__device__ __forceinline__ float dot8f(const u32x4 w, const float* x, float acc) {
  acc = fmaf(bflo(w.x), x[0], acc);
  acc = fmaf(bfhi(w.x), x[1], acc);
  acc = fmaf(bflo(w.y), x[2], acc);
  acc = fmaf(bfhi(w.y), x[3], acc);
  acc = fmaf(bflo(w.z), x[4], acc);
  acc = fmaf(bfhi(w.z), x[5], acc);
  acc = fmaf(bflo(w.w), x[6], acc);
  acc = fmaf(bfhi(w.w), x[7], acc);
  return acc;
}
__device__ __forceinline__ double dot8a(const u32x4 w, const double* x, double acc) { return dot8d(w, x, acc); }
__device__ __forceinline__ float dot8a(const u32x4 w, const float* x, float acc) { return dot8f(w, x, acc); }

// Value the optimizer must treat as unknown (an empty asm that claims to modify it): derived
// quantities cannot be hoisted or CSE'd across the point where it is produced.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Global-address-space view of a device pointer. Loads through it compile to global_load
// (counted by vmcnt only); loads through a generic pointer compile to flat_load, which also
// counts against lgkmcnt, so every LDS wait would also wait for the weight prefetches.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}
// Constant-address-space view of a table that no wave writes during the launch (the layer
// pointer table, the head / embedding pointer arrays): loads at a wave-uniform address become
// scalar loads, which are counted by lgkmcnt and so never wait behind the vector-memory queue
// of in-flight weight prefetches.
template <class T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}
// 1 / sqrt(x) for normal x > 0 in f64: the hardware estimate (about 2^-23 relative) refined by
// two Newton steps y += y (1/2 - x y^2 / 2); the result is within a few ulps of the correctly
// rounded 1.0 / sqrt(x), at a fraction of the latency of the IEEE square root and division.
__device__ __forceinline__ double rsqrt_d(double x) {
  double y = __builtin_amdgcn_rsq(x);
  const double h = 0.5 * x;
  y = fma(y, fma(-(h * y), y, 0.5), y);
  y = fma(y, fma(-(h * y), y, 0.5), y);
  return y;
}
// 1 / x for normal x > 0 in f64: the hardware estimate refined by two Newton steps
// y += y (1 - x y); within a few ulps of the correctly rounded 1.0 / x.
__device__ __forceinline__ double rcp_d(double x) {
  double y = __builtin_amdgcn_rcp(x);
  y = fma(y, fma(-x, y, 1.0), y);
  y = fma(y, fma(-x, y, 1.0), y);
  return y;
}
// 1 / sqrt(x) for normal x > 0 in f32: the hardware estimate refined by one Newton step.
__device__ __forceinline__ float rsqrt_f(float x) {
  float y = __builtin_amdgcn_rsqf(x);
  const float h = 0.5f * x;
  return fmaf(y, fmaf(-(h * y), y, 0.5f), y);
}
// 1 / x for normal x > 0 in f32: the hardware estimate refined by one Newton step.
__device__ __forceinline__ float rcp_f(float x) {
  float y = __builtin_amdgcn_rcpf(x);
  return fmaf(y, fmaf(-x, y, 1.0f), y);
}
__device__ __forceinline__ double rsqrt_a(double x) { return rsqrt_d(x); }
__device__ __forceinline__ float rsqrt_a(float x) { return rsqrt_f(x); }
__device__ __forceinline__ double exp_a(double x) { return exp(x); }
__device__ __forceinline__ float exp_a(float x) { return __expf(x); }

// store through the global address space (a global_store, not a flat one)
template <class T>
__device__ __forceinline__ void gput(T* p, T v) {
  *(__attribute__((address_space(1))) T*)p = v;
}
__device__ __forceinline__ u32x4 ldw(const bf16_t* p) { return *gmem(reinterpret_cast<const u32x4*>(p)); }
__device__ __forceinline__ float ldbf(const bf16_t* p) { return bf2f(*gmem(p)); }
__device__ __forceinline__ u32x4 ldw_nt(const bf16_t* p) {
  return __builtin_nontemporal_load(gmem(reinterpret_cast<const u32x4*>(p)));
}

// ---------------------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------------------
// Cross-lane exchange partners used by the group reductions (all VALU, no LDS traffic):
//   step 0: quad_perm [1,0,3,2]   (lane ^ 1)
//   step 1: quad_perm [2,3,0,1]   (lane ^ 2)
//   step 2: row_half_mirror       (lane i <-> 7 - i within 8 lanes)
//   step 3: row_mirror            (lane i <-> 15 - i within 16 lanes)
//   step 4: v_permlane16_swap     (lane i <-> i + 16 within 32 lanes)
//   step 5: v_permlane32_swap     (lane i <-> i + 32)
// After step k every lane of its 2^(k+1)-lane group holds the same combined value.
template <int STEP>
__device__ __forceinline__ uint32_t xlane(uint32_t v) {
  if constexpr (STEP == 0) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
  else if constexpr (STEP == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
  else if constexpr (STEP == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);
  else if constexpr (STEP == 3) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
  else if constexpr (STEP == 4) { auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false); return r[0] ^ r[1] ^ v; }
  else { auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false); return r[0] ^ r[1] ^ v; }
}
template <int STEP>
__device__ __forceinline__ float xlane_f(float v) { return __uint_as_float(xlane<STEP>(__float_as_uint(v))); }
template <int STEP>
__device__ __forceinline__ double xlane_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t r = (uint64_t)xlane<STEP>((uint32_t)u) | ((uint64_t)xlane<STEP>((uint32_t)(u >> 32)) << 32);
  return __builtin_bit_cast(double, r);
}
// lane K of each group of 4 lanes, to all 4 (DPP quad_perm [K, K, K, K])
template <int K>
__device__ __forceinline__ double quad_bcast_d(double v) {
  constexpr int ctrl = K | (K << 2) | (K << 4) | (K << 6);
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)u, ctrl, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), ctrl, 0xF, 0xF, false);
  return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}
// a pair of values reduced together (e.g. a gate and an up projection of one row)
template <class T> struct pair2 { T a, b; };
template <class T>
__device__ __forceinline__ pair2<T> operator+(pair2<T> x, pair2<T> y) { return pair2<T>{x.a + y.a, x.b + y.b}; }
template <int STEP, typename T>
__device__ __forceinline__ T xlane_t(T v) {
  if constexpr (std::is_same_v<T, double>) return xlane_d<STEP>(v);
  else if constexpr (std::is_same_v<T, float>) return xlane_f<STEP>(v);
  else return T{xlane_t<STEP>(v.a), xlane_t<STEP>(v.b)};
}

// Sum / max over aligned groups of WIDTH lanes (WIDTH in {16, 32, 64}); every lane of a group
// receives the group's result.
template <int WIDTH, typename T>
__device__ __forceinline__ T group_sum(T v) {
  v += xlane_t<0>(v);
  v += xlane_t<1>(v);
  v += xlane_t<2>(v);
  v += xlane_t<3>(v);
  if constexpr (WIDTH >= 32) v += xlane_t<4>(v);
  if constexpr (WIDTH >= 64) v += xlane_t<5>(v);
  return v;
}
template <int WIDTH, typename T>
__device__ __forceinline__ T group_max(T v) {
  T u;
  u = xlane_t<0>(v); v = u > v ? u : v;
  u = xlane_t<1>(v); v = u > v ? u : v;
  u = xlane_t<2>(v); v = u > v ? u : v;
  u = xlane_t<3>(v); v = u > v ? u : v;
  if constexpr (WIDTH >= 32) { u = xlane_t<4>(v); v = u > v ? u : v; }
  if constexpr (WIDTH >= 64) { u = xlane_t<5>(v); v = u > v ? u : v; }
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) { return group_sum<64>(v); }
// Reduce-scatter sum of N values (N a power of two) over aligned groups of 2^(STEP+1) lanes.
// At each of the first log2(N) steps the lane keeps half of its values (the lower half when
// its STEP bit is 0) and adds the partner's copy of that half, received in one exchange per
// kept value; the remaining steps sum the single value left. On return every lane holds the
// group total of value k = sum over the split steps s of bit_s(lane) * (count at s) / 2,
// e.g. N = 4 over 64 lanes: k = 2 * bit5 + bit4. The exchange partners are those of xlane.
template <int STEP, int N, typename T>
__device__ __forceinline__ T rs_sum(const T (&c)[N], int lane) {
  if constexpr (STEP < 0) {
    return c[0];
  } else if constexpr (N == 1) {
    T v = c[0];
    v = v + xlane_t<STEP>(v);
    if constexpr (STEP > 0) {
      const T o[1] = {v};
      return rs_sum<STEP - 1, 1>(o, lane);
    } else {
      return v;
    }
  } else {
    constexpr int H = N / 2;
    const bool hi = (lane >> STEP) & 1;
    T o[H];
#pragma unroll
    for (int j = 0; j < H; ++j) {
      const T send = hi ? c[j] : c[H + j];
      const T keep = hi ? c[H + j] : c[j];
      o[j] = keep + xlane_t<STEP>(send);
    }
    return rs_sum<STEP - 1, H>(o, lane);
  }
}

// group_sum / group_max of N independent values, step by step across all of them, so the
// cross-lane moves of one value fill the DPP wait states of the others (same results).
template <int WIDTH, int N, typename T>
__device__ __forceinline__ void group_sum_n(T (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += xlane_t<0>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += xlane_t<1>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += xlane_t<2>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += xlane_t<3>(v[i]);
  if constexpr (WIDTH >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += xlane_t<4>(v[i]);
  }
  if constexpr (WIDTH >= 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += xlane_t<5>(v[i]);
  }
}

// ---------------------------------------------------------------------------------------
// exchange slots
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t slot_pack(float v, uint32_t tag) {
  return ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}
// XCD-local publish: a plain 8-byte store (lands in the XCD's L2).
__device__ __forceinline__ void put_local(uint64_t* p, float v, uint32_t tag) {
  *p = slot_pack(v, tag);
}
// cross-XCD publish: write-through to memory (sc1).
__device__ __forceinline__ void put_cross(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, slot_pack(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct ErrCtl {
  uint32_t* err;
  uint32_t spin_cap;
};

__device__ __forceinline__ bool err_set(const ErrCtl& c) {
  return __hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

// Poll `n` slots (n even, buf 16-byte aligned) until every tag equals `tag`; store the values
// to dst[0..n). Executed by one wave. 16-byte sc1 buffer loads fetch two slots each; every
// 8-byte half carries its own tag. Returns false (and latches the error word) on timeout.
template <int MAXPAIRS_PER_LANE>
__device__ bool poll_slots(const uint64_t* buf, int n, uint32_t tag, float* dst, const ErrCtl& c) {
  const int lane = threadIdx.x & 63;
  const int npair = n >> 1;
  __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(buf), (short)0, n * 8, 0x00020000);
  uint32_t pending = 0;
#pragma unroll
  for (int k = 0; k < MAXPAIRS_PER_LANE; ++k)
    if (lane + 64 * k < npair) pending |= 1u << k;
  uint32_t spins = 0;
  for (;;) {
    u32x4 v[MAXPAIRS_PER_LANE];
#pragma unroll
    for (int k = 0; k < MAXPAIRS_PER_LANE; ++k)
      if (pending & (1u << k)) v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane + 64 * k) * 16, 0, 16);
#pragma unroll
    for (int k = 0; k < MAXPAIRS_PER_LANE; ++k) {
      if ((pending & (1u << k)) && v[k].y == tag && v[k].w == tag) {
        const int i = (lane + 64 * k) * 2;
        dst[i] = __uint_as_float(v[k].x);
        dst[i + 1] = __uint_as_float(v[k].z);
        pending &= ~(1u << k);
      }
    }
    if (__ballot(pending != 0u) == 0ull) return true;
    ++spins;
    if ((spins & 63u) == 0u && (spins > c.spin_cap || err_set(c))) {
      if (lane == 0) atomicOr(c.err, 1u);
      return false;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Philox-4x64-10 (Salmon et al., SC'11) and the sampler's uniform draw.
// Stream layout: key = (seed, "QTTSAFMP"), counter = (vocab_id / 4, frame_step, group, 0),
// word = vocab_id % 4, u = ((word >> 12) + 0.5) * 2^-52: the sum is exact (53 bits), so
// u lies strictly inside (0, 1) for every word.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void philox4x64_10(uint64_t c[4], uint64_t k0, uint64_t k1) {
  const uint64_t M0 = 0xD2E7470EE14C6C93ull, M1 = 0xCA5A826395121157ull;
  const uint64_t W0 = 0x9E3779B97F4A7C15ull, W1 = 0xBB67AE8584CAA73Bull;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) { k0 += W0; k1 += W1; }
    const uint64_t lo0 = M0 * c[0], hi0 = __umul64hi(M0, c[0]);
    const uint64_t lo1 = M1 * c[2], hi1 = __umul64hi(M1, c[2]);
    const uint64_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
  }
}
__device__ __forceinline__ double sampler_uniform(uint64_t seed, int frame_step, int group, int vid) {
  uint64_t c[4] = {(uint64_t)(vid >> 2), (uint64_t)(uint32_t)frame_step, (uint64_t)(uint32_t)group, 0ull};
  philox4x64_10(c, seed, 0x5154545341464D50ull);
  return ((double)(c[vid & 3] >> 12) + 0.5) * (1.0 / 4503599627370496.0);
}

// Order-preserving map float -> uint32 (larger float, larger key).
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

}  // namespace qtts
