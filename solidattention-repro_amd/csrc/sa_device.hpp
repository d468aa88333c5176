// sa_device.hpp — device-side helpers shared by the gfx950 kernels of the
// KV-cache decode hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sa {

// ---- geometry ------------------------------------------------------------
// A page holds kPageTokens tokens.  A token is [K: Hkv x D][V: Hkv x D] FP16,
// the reference's token-major K/V-interleaved format (backend.hpp:18-31 of
// the reference), so a 32-token page at Hkv=8, D=128 is 128 KiB and a block
// read from the host store lands in a page with one copy.
constexpr int kPageTokens = 32;
constexpr int kWave = 64;

// Status bits a kernel ORs into an optional device status word.
enum StatusBits : int32_t {
  kStatusBadPage = 1,       // page id outside [0, num_pages)
  kStatusBadBlock = 2,      // logical block outside the table / sealed range
  kStatusBadLength = 4,     // seq_len / sealed inconsistent
  kStatusCapacity = 8,      // representative or table capacity exceeded
  kStatusBadBudget = 16,    // per-sequence budget outside [init + local, sel_stride]
};

__device__ inline void flag_status(int32_t* status, int32_t bits) {
  if (status) atomicOr(status, bits);
}

// ---- values handed between workgroups -------------------------------------
// A workgroup that hands values to another (possibly on another XCD, whose
// L2 is not shared) stores them with agent-scope atomic stores and the
// receiver reads them with agent-scope atomic loads.  An agent-scope fence
// (__threadfence) would write back and invalidate the whole L2 of the XCD.
template <class T>
__device__ inline void store_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ inline T load_agent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The last of `arrivals` workgroups to reach the counter gets true and
// resets it to zero; every thread calls it after its handed-over stores.
__device__ inline bool last_arrival(int32_t* ctr, int arrivals, int* s_last) {
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == arrivals - 1;
    if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = last;
  }
  __syncthreads();
  return *s_last;
}

// ---- FP16 ------------------------------------------------------------------
// v_cvt_f32_f16 is exact for every FP16 input (subnormals included), so it
// equals the reference's bit-level decode (attention_reference.cpp:30-53).
__device__ inline float h2f(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// v_cvt_f16_f32 under the default MODE (round to nearest even): the
// reference's device append conversion (cvt.rn.f16.f32,
// qwen_layer_main.cpp:277-278).
__device__ inline uint16_t f2h_rne(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// Low / high half of a packed pair as fp32.
__device__ inline float lo_h2f(uint32_t w) { return h2f(static_cast<uint16_t>(w & 0xffffu)); }
__device__ inline float hi_h2f(uint32_t w) { return h2f(static_cast<uint16_t>(w >> 16)); }

// ---- the received-mass order of the InfLLM builder ---------------------------
// Keys are ranked by received mass, greater first, equal masses in token
// order (the reference's std::stable_sort with a > b, selection.cpp:71-76).
// That comparator leaves NaN unordered, where std::stable_sort has no defined
// result; here NaN ranks after every number and NaNs keep token order, so
// that the rank of key j, #{k : before(m_k, m_j)} + #{k < j : tied(m_k, m_j)},
// is a bijection for every input.  Numbers rank exactly as with a > b.
__device__ inline bool mass_before(float a, float b) { return (a > b) || (a == a && b != b); }
__device__ inline bool mass_tied(float a, float b) { return !(a > b) && !(b > a) && ((a == a) == (b == b)); }

// ---- streaming loads ---------------------------------------------------------
// Non-temporal 16-byte load: data read once per step (KV pages,
// representatives) is streamed past the caches.  On MI355X this lifts the
// sparse attention's page reads from 5.3 to 6.1 TB/s.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ inline uint4 load_stream16(const void* a) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(a));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ inline float load_stream_f32(const float* a) { return __builtin_nontemporal_load(a); }

// ---- cross-lane reductions (DPP, 16-lane rows) --------------------------
// DPP controls (gfx9): quad_perm, row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int Ctrl>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), Ctrl, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
// After the two quad steps all lanes of a quad hold the same value, so the
// half-row and row mirrors act as exchanges with the other quad / half.
__device__ inline float row16_sum(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave: shifts by 1, 2, 4, 8
// within each 16-lane row, then row 0's last lane into rows 1 and 3 and lane
// 31 into rows 2 and 3 (row_bcast).  Lanes whose source lies outside the
// row, and rows the row mask leaves out, add 0.
template <int Ctrl, int RowMask>
__device__ inline uint32_t dpp_or_zero(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), Ctrl, RowMask, 0xF, false));
}

__device__ inline uint32_t wave_prefix_sum(uint32_t v) {
  v += dpp_or_zero<0x111, 0xF>(v);  // row_shr:1
  v += dpp_or_zero<0x112, 0xF>(v);  // row_shr:2
  v += dpp_or_zero<0x114, 0xF>(v);  // row_shr:4
  v += dpp_or_zero<0x118, 0xF>(v);  // row_shr:8
  v += dpp_or_zero<0x142, 0xA>(v);  // row_bcast:15
  v += dpp_or_zero<0x143, 0xC>(v);  // row_bcast:31
  return v;
}

__device__ inline float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// ---- synthetic data (bit-identical to the host generator) ----------------
// splitmix64 output function.
__device__ __host__ inline uint64_t mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Irwin-Hall(4) normal: exact integer sum of four 16-bit uniforms, centred,
// times 1/sigma in one fp32 multiply.
__device__ inline float synth_normal(uint64_t seed_mixed, uint64_t index) {
  const uint64_t h = mix64(seed_mixed ^ index);
  const int32_t sum = static_cast<int32_t>(h & 0xffffu) + static_cast<int32_t>((h >> 16) & 0xffffu) +
                      static_cast<int32_t>((h >> 32) & 0xffffu) + static_cast<int32_t>(h >> 48) - 131070;
  return __fmul_rn(static_cast<float>(sum), 2.6428937e-05f);
}

}  // namespace sa
