// Exchange-slot polling shared by the decode kernels: a wave polls tagged {f32 value, u32 tag}
// slots of a workspace through one buffer descriptor (L2-coherent sc1 loads) into registers or LDS.
#pragma once
#include "qtts_common.h"

namespace qtts {

struct Poll {
  __amdgpu_buffer_rsrc_t rs;   // covers the whole workspace
  const void* base;
  ErrCtl ec;
};

__device__ __forceinline__ uint32_t ws_off(const Poll& P, const void* p) {
  return (uint32_t)(reinterpret_cast<const char*>(p) - reinterpret_cast<const char*>(P.base));
}

// Poll npair 16-byte pairs (two tagged slots each) into registers: pair k of this lane, index
// i = lane + 64 k (i < npair), lives at byte offset off(i) of the workspace and lands in
// out[2 k], out[2 k + 1]. Returns false on timeout (error word set).
template <int MAXP, typename OffF>
__device__ bool poll_regs(const Poll& P, int npair, uint32_t tag, float (&out)[2 * MAXP], OffF off) {
  const int lane = opaque((int)threadIdx.x & 63);   // keeps slot offsets from being hoisted and spilled
  uint32_t valid = 0;
#pragma unroll
  for (int k = 0; k < MAXP; ++k)
    if (lane + 64 * k < npair) valid |= 1u << k;
  uint32_t pending = valid;
  uint32_t spins = 0;
  auto check = [&](const u32x4 (&v)[MAXP]) {
#pragma unroll
    for (int k = 0; k < MAXP; ++k) {
      if ((pending & (1u << k)) && v[k].y == tag && v[k].w == tag) {
        out[2 * k] = __uint_as_float(v[k].x);
        out[2 * k + 1] = __uint_as_float(v[k].z);
        pending &= ~(1u << k);
      }
    }
    return __ballot(pending != 0u) == 0ull;
  };
  auto timed_out = [&]() {
    ++spins;
    if ((spins & 63u) == 0u && (spins > P.ec.spin_cap || err_set(P.ec))) {
      if (lane == 0) atomicOr(P.ec.err, 1u);
      return true;
    }
    return false;
  };
  if constexpr (MAXP <= 17) {
    // NBAT batches in flight: the next batch is issued before the oldest one is checked, so a
    // slot is seen about 1 / NBAT of a load latency after it lands instead of a whole one.
    // Every batch has the same loads (lanes without a slot re-read slot 0), so the wait for
    // the oldest batch is an exact vmcnt.
    constexpr int NBAT = MAXP <= 2 ? 4 : (MAXP <= 4 ? 3 : 2);
    u32x4 vb[NBAT][MAXP];
    auto issue = [&](u32x4 (&v)[MAXP]) {
#pragma unroll
      for (int k = 0; k < MAXP; ++k)
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(P.rs, off((valid >> k) & 1u ? lane + 64 * k : 0), 0, 16);
    };
#pragma unroll
    for (int b = 0; b < NBAT - 1; ++b) issue(vb[b]);
    for (;;) {
#pragma unroll
      for (int b = 0; b < NBAT; ++b) {
        issue(vb[(b + NBAT - 1) % NBAT]);
        if (check(vb[b])) return true;
      }
      if (timed_out()) return false;
    }
  } else {
    // one round in flight; every load issued unconditionally (a load under a branch makes the
    // compiler wait for it before issuing the next)
    for (;;) {
      u32x4 v[MAXP];
#pragma unroll
      for (int k = 0; k < MAXP; ++k)
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(P.rs, off((valid >> k) & 1u ? lane + 64 * k : 0), 0, 16);
      if (check(v)) return true;
      if (timed_out()) return false;
    }
  }
}
// Read npair 16-byte pairs into registers (pair k of this lane: i = lane + 64 k < npair) until
// every tag matches, one round of loads in flight: for data that has (nearly all) arrived, which
// a batched poll would fetch several times over. Every load of a round is issued
// unconditionally (pairs already taken and lanes without a pair re-read a valid slot): a load
// under a branch makes the compiler wait for it before issuing the next, serialising the round.
template <int MAXP, typename OffF>
__device__ __forceinline__ bool read_pairs(const Poll& P, int npair, uint32_t tag, float (&out)[2 * MAXP], OffF off) {
  const int lane = opaque((int)threadIdx.x & 63);
  uint32_t pending = 0;
#pragma unroll
  for (int k = 0; k < MAXP; ++k)
    if (lane + 64 * k < npair) pending |= 1u << k;
  const uint32_t valid = pending;
  uint32_t spins = 0;
  for (;;) {
    u32x4 v[MAXP];
#pragma unroll
    for (int k = 0; k < MAXP; ++k)
      v[k] = __builtin_amdgcn_raw_buffer_load_b128(P.rs, off((valid >> k) & 1u ? lane + 64 * k : 0), 0, 16);
#pragma unroll
    for (int k = 0; k < MAXP; ++k) {
      if ((pending & (1u << k)) && v[k].y == tag && v[k].w == tag) {
        out[2 * k] = __uint_as_float(v[k].x);
        out[2 * k + 1] = __uint_as_float(v[k].z);
        pending &= ~(1u << k);
      }
    }
    if (__ballot(pending != 0u) == 0ull) return true;
    ++spins;
    if ((spins & 63u) == 0u && (spins > P.ec.spin_cap || err_set(P.ec))) {
      if (lane == 0) atomicOr(P.ec.err, 1u);
      return false;
    }
  }
}
// Poll npair pairs into LDS: pair i to dst[2 i], dst[2 i + 1].
template <int MAXP, typename OffF>
__device__ bool poll_pairs(const Poll& P, int npair, uint32_t tag, float* dst, OffF off) {
  float v[2 * MAXP];
  const bool ok = poll_regs<MAXP>(P, npair, tag, v, off);
  const int lane = opaque((int)threadIdx.x & 63);
#pragma unroll
  for (int k = 0; k < MAXP; ++k)
    if (lane + 64 * k < npair) *reinterpret_cast<float2*>(dst + 2 * (lane + 64 * k)) = make_float2(v[2 * k], v[2 * k + 1]);
  return ok;
}
// contiguous n slots (n even) starting at p
template <int MAXP>
__device__ __forceinline__ bool poll_vec(const Poll& P, const uint64_t* p, int n, uint32_t tag, float* dst) {
  const uint32_t o = ws_off(P, p);
  return poll_pairs<MAXP>(P, n >> 1, tag, dst, [o](int i) { return o + 16u * (uint32_t)i; });
}
// contiguous n slots (n even, up to MAXV) into LDS, in pieces of 1024 slots (8 pairs per lane):
// each piece keeps two batches of 8 loads in flight, and no more registers than that are held
__device__ __forceinline__ bool poll_vec_long(const Poll& P, const uint64_t* p, int n, uint32_t tag, float* dst) {
  bool ok = true;
  for (int s0 = 0; s0 < n; s0 += 1024) {
    const int m = n - s0 < 1024 ? n - s0 : 1024;
    ok = poll_vec<8>(P, p + s0, m, tag, dst + s0) && ok;
  }
  return ok;
}
// contiguous 1024 slots into registers: this lane gets elements 2 (lane + 64 k) + {0, 1}
__device__ __forceinline__ bool poll_vec_regs(const Poll& P, const uint64_t* p, uint32_t tag, float (&out)[16]) {
  const uint32_t o = ws_off(P, p);
  return poll_regs<8>(P, HID / 2, tag, out, [o](int i) { return o + 16u * (uint32_t)i; });
}

// A 1024-vector published by the 32 workgroups of an XCD, workgroup j writing rows
// [32 j, 32 j + 32) as 16 pairs from one store instruction: lanes 0..31 poll the last pair of
// producer `lane` until all 32 have landed, then every pair is read once (lane gets elements
// 2 (lane + 64 k) + {0, 1}). Polling one pair per producer instead of all 512 keeps the eight
// waves' polls from filling the CU's memory pipeline.
__device__ __forceinline__ bool gather1024(const Poll& P, const uint64_t* p, uint32_t tag, float (&out)[16]) {
  const uint32_t o = ws_off(P, p);
  float pr[2];
  if (!poll_regs<1>(P, WPX, tag, pr, [o](int i) { return o + 16u * (16u * (uint32_t)i + 15u); })) return false;
  return read_pairs<8>(P, HID / 2, tag, out, [o](int i) { return o + 16u * (uint32_t)i; });
}

// Workgroup barrier: makes LDS data one wave wrote visible to the others. Every wave of the
// workgroup must reach each barrier the same number of times.
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

}  // namespace qtts
