// schedule.hpp — workgroup order for lists of very different lengths.
//
// A launch with one workgroup per (list, chunk) runs in dispatch order; when
// the long lists' chunks come last, they run while most compute units sit
// idle.  build_list_schedule(), run by one 1024-thread workgroup before such
// a launch, counting-sorts the lists by a length key (4096 bins in LDS,
// longest first; the order within a bin is arbitrary) and writes, for every
// workgroup w of the launch (dispatch order), the list and chunk it takes:
//   sched[w] = list (-1: nothing), sched[slots + w] = chunk,
// a list's chunks consecutive.  The consumers read their assignment from it;
// what each chunk computes does not depend on the order.
#pragma once

#include "sa_device.hpp"

namespace sa {
namespace {

constexpr int kSchedMaxLists = 4096;
constexpr int kSchedBins = 4096;
constexpr int kSchedThreads = 1024;
constexpr int kSchedPer = kSchedMaxLists / kSchedThreads;

// Exclusive prefix sum over the workgroup's threads (in thread order).
__device__ inline int sched_scan(int v, int* wave_sums) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  int incl = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int t = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += t;
  }
  if (lane == kWave - 1) wave_sums[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kSchedThreads / kWave ? wave_sums[lane] : 0;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int t = __shfl_up(w, off, kWave);
      if (lane >= off) w += t;
    }
    if (lane < kSchedThreads / kWave) wave_sums[lane] = w;  // inclusive over waves
  }
  __syncthreads();
  const int before = wave > 0 ? wave_sums[wave - 1] : 0;
  __syncthreads();  // wave_sums reusable
  return before + incl - v;
}

// n lists (<= kSchedMaxLists), slots workgroups in the launch (>= the sum of
// the lists' chunks).  info(l, key, chunks) gives list l's length key in
// [0, kSchedBins) and its chunk count (>= 1).  Called by every thread of a
// kSchedThreads-thread workgroup.
template <class Info>
__device__ inline void build_list_schedule(int n, int64_t slots, int32_t* sched, Info info) {
  const int tid = threadIdx.x;
  __shared__ int hist[kSchedBins];
  __shared__ int sorted[kSchedMaxLists];
  __shared__ int nch[kSchedMaxLists];
  __shared__ int wave_sums[kSchedThreads / kWave];
  __shared__ int s_used;
  for (int i = tid; i < kSchedBins; i += kSchedThreads) hist[i] = 0;
  __syncthreads();
  int bin[kSchedPer];
#pragma unroll
  for (int k = 0; k < kSchedPer; ++k) {
    const int l = tid + k * kSchedThreads;
    bin[k] = -1;
    if (l < n) {
      int key = 0, chunks = 1;
      info(l, key, chunks);
      key = key < 0 ? 0 : (key > kSchedBins - 1 ? kSchedBins - 1 : key);
      nch[l] = chunks < 1 ? 1 : chunks;
      bin[k] = kSchedBins - 1 - key;  // longest in bin 0
      atomicAdd(&hist[bin[k]], 1);
    }
  }
  __syncthreads();
  // bins -> first sorted position (4 bins per thread)
  constexpr int kBinsPer = kSchedBins / kSchedThreads;
  int hs[kBinsPer];
  int hsum = 0;
#pragma unroll
  for (int i = 0; i < kBinsPer; ++i) {
    hs[i] = hist[tid * kBinsPer + i];
    hsum += hs[i];
  }
  int off = sched_scan(hsum, wave_sums);
#pragma unroll
  for (int i = 0; i < kBinsPer; ++i) {
    hist[tid * kBinsPer + i] = off;
    off += hs[i];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kSchedPer; ++k) {
    const int l = tid + k * kSchedThreads;
    if (l < n) sorted[atomicAdd(&hist[bin[k]], 1)] = l;
  }
  __syncthreads();
  // first workgroup of each sorted list (kSchedPer consecutive lists per thread)
  int c[kSchedPer];
  int csum = 0;
#pragma unroll
  for (int k = 0; k < kSchedPer; ++k) {
    const int i = tid * kSchedPer + k;
    c[k] = i < n ? nch[sorted[i]] : 0;
    csum += c[k];
  }
  int w = sched_scan(csum, wave_sums);
#pragma unroll
  for (int k = 0; k < kSchedPer; ++k) {
    const int i = tid * kSchedPer + k;
    if (i < n) {
      const int l = sorted[i];
      for (int zz = 0; zz < c[k]; ++zz) {
        sched[w + zz] = l;
        sched[slots + w + zz] = zz;
      }
    }
    w += c[k];
  }
  // the workgroups past the last chunk have nothing to do
  if (tid == kSchedThreads - 1) s_used = w;  // every list's chunks
  __syncthreads();
  for (int64_t e = s_used + tid; e < slots; e += kSchedThreads) sched[e] = -1;
}

}  // namespace
}  // namespace sa
