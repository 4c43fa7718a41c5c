// End-to-end two-stage top-k (YOLO26 / v10 heads), bit-exact with
// CpuEndToEnd.SelectPt / SelectOnnx (src/SimdYolo/CpuEndToEnd.cs:26-241).
//
// Every candidate has a unique 64-bit key: an order-preserving image of its
// score (-0 ties +0; NaN lowest under PT rules, highest under ONNX rules)
// above the inverted tie index, so "larger key" is exactly the reference's
// order (score descending, tie index ascending).  Kernels:
//   * topk_class_pass_kernel, over the whole GPU: per anchor the class
//     maximum (.NET Max: NaN propagates) as the stage-1 key, and the anchor's
//     four best classes as packed 32-bit records (truncated key, class).  A
//     workgroup owns 64 anchors of one image; its four waves each scan a
//     quarter of the classes with coalesced row reads and merge in LDS;
//   * topk_select_kernel, one 1024-thread workgroup per image.  An MSB-first
//     radix select finds the k-th largest key; digit passes run until the
//     prefix isolates exactly k keys.  Stage 1 ranks the anchors.  Their keys
//     stay in registers when the image has at most 33 * 1024 anchors: the
//     radix runs over key - (lowest score << 32), whose top bit follows from
//     the scores' minimum and maximum, with 11-bit digits (one LDS atomic per
//     key per pass; usually one pass).  Larger images re-read the keys from
//     global memory on every pass (8-bit digits, the shared leading bits found
//     by one OR reduction).  Under PT rules only the set matters; under ONNX
//     rules the k keys at or above the threshold are each placed by their
//     rank.  Each selected anchor owns a pair scoring exactly its stage-1 key,
//     so no pair scoring below the stage-1 threshold can be among the k best:
//     stage 2 takes its candidates from the anchors' records (re-reading the
//     exact score of each record that may reach the bound, and an anchor's
//     full class column when its fourth record may).  A pair's tie index is
//     anchor * nc + class under PT rules and stage-1 rank * nc + class under
//     ONNX rules, so the selected anchors need no order under PT rules.  The
//     listed candidates (at least k, at most 1024) are ranked among
//     themselves by a counting sort on their top score bits; the workgroup
//     then writes the first six fields of the image's [k, 6 + extra] rows;
//   * topk_extras_kernel, over the whole GPU, when the head has extra
//     channels: those fields of each row, scattered gathers by the picks.
#include <cstddef>
#include <cstdint>
#include <mutex>

#include "sy_internal.h"

namespace sy {

constexpr int kTkThreads = 1024;
constexpr int kTkCap = 32768;      // candidates per stage held in LDS
constexpr int kTkMaxAnchors = 1 << 24;  // stage-1 keys beyond kTkCap stay in global memory
constexpr int kTkMaxK = 1024;
constexpr int kTkList = 1024;      // stage-2 candidates compacted under the stage-1 bound
constexpr int kTkGroup = 64;       // anchors per workgroup of the class pass
constexpr int kTkRec = 4;          // best classes kept per anchor
constexpr int kTkScan = 20;        // class rows a lane loads before using them (80 classes: one batch per wave)
constexpr int kTkRecClasses = 127; // class counts the 7-bit class field of a record holds

// An anchor's four best classes as packed records, largest first: the score
// key's upper 25 bits above 127 - class, so a larger record is a larger
// (truncated) key or, among equal truncated keys, a smaller class; 0 is an
// empty slot (a filled record is at least 1).  Truncation only widens what
// stage 2 must look at: a class with key >= bound has record >> 7 >=
// bound >> 7, and stage 2 re-reads the exact score of every listed record.
struct TopRec {
  uint32_t r[kTkRec];
};

__device__ __forceinline__ uint32_t score_key(float f, bool onnx) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return onnx ? 0xffffffffu : 0u;  // NaN
  if (u == 0x80000000u) u = 0u;                                          // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long full_key(uint32_t k32, uint32_t idx) {
  return ((unsigned long long)k32 << 32) | (unsigned long long)(0xffffffffu - idx);
}

// Inserts record x into the list (descending, records unique per anchor),
// which keeps the four largest records in order: slot p becomes the median
// of the old slots p - 1 and p and x (one v_med3_u32 each; updated from the
// last slot down, so in place), slot 0 the max.  x = 0 (an empty record)
// leaves the list unchanged.
__device__ __forceinline__ void rec_insert(uint32_t (&rk)[kTkRec], uint32_t x) {
#pragma unroll
  for (int p = kTkRec - 1; p >= 1; --p) rk[p] = max(min(rk[p - 1], rk[p]), min(max(rk[p - 1], rk[p]), x));
  rk[0] = max(rk[0], x);
}

__device__ __forceinline__ uint32_t make_record(uint32_t key, int cls) {
  return (key & ~127u) | (uint32_t)(127 - cls);
}

__global__ __launch_bounds__(256) void topk_class_pass_kernel(const float* __restrict__ head, int channels,
                                                              int anchors, int nc, int onnx,
                                                              uint32_t* __restrict__ keys,
                                                              TopRec* __restrict__ recs) {
  __shared__ uint32_t pm[4][kTkGroup], pn[4][kTkGroup];
  __shared__ uint32_t pk[4][kTkRec][kTkGroup];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int a = blockIdx.x * kTkGroup + lane;
  const bool ox = onnx != 0;
  const float* rows = head + ((long long)b * channels + 4) * anchors;  // the class rows of image b
  const int per = (nc + 3) / 4, c0 = wave * per, c1 = min(nc, c0 + per);
  // The anchor's maximum is tracked on the order-preserving keys (-0 ties
  // +0): kmax, and kmin, which is 0 exactly when a class score is NaN under
  // PyTorch rules (NaN's key); under ONNX rules NaN has the largest key.
  uint32_t kmax = 0x007fffffu, kmin = 0xffffffffu;  // kmax starts at the key of -inf
  const bool recs_on = nc <= kTkRecClasses;
  uint32_t rk[kTkRec];
#pragma unroll
  for (int p = 0; p < kTkRec; ++p) rk[p] = 0u;
  if (a < anchors) {
    // A wave's quarter of the classes (20 rows for 80 classes) is loaded in
    // one batch before any is used.  Rows past the end re-read the last one:
    // that changes neither extreme, and its record is replaced by the empty
    // one (no per-row branch).  Offsets within an image fit 32 bits.
    for (int cb = c0; cb < c1; cb += kTkScan) {
      float v[kTkScan];
#pragma unroll
      for (int i = 0; i < kTkScan; ++i) v[i] = rows[(unsigned)min(cb + i, c1 - 1) * (unsigned)anchors + (unsigned)a];
#pragma unroll
      for (int i = 0; i < kTkScan; ++i) {
        const uint32_t k = score_key(v[i], ox);
        kmax = max(kmax, k);
        kmin = min(kmin, k);
        if (recs_on) rec_insert(rk, cb + i < c1 ? make_record(k, cb + i) : 0u);
      }
    }
  }
  pm[wave][lane] = kmax;
  pn[wave][lane] = kmin;
#pragma unroll
  for (int p = 0; p < kTkRec; ++p) pk[wave][p][lane] = rk[p];
  __syncthreads();
  if (wave != 0 || a >= anchors) return;
  for (int w = 1; w < 4; ++w) {
    kmax = max(kmax, pm[w][lane]);
    kmin = min(kmin, pn[w][lane]);
#pragma unroll
    for (int p = 0; p < kTkRec; ++p) rec_insert(rk, pk[w][p][lane]);
  }
  const long long o = (long long)b * anchors + a;
  keys[o] = (!ox && kmin == 0u) ? 0u : kmax;  // PyTorch rules: a NaN class makes the maximum NaN (key 0)
  TopRec r;
#pragma unroll
  for (int p = 0; p < kTkRec; ++p) r.r[p] = rk[p];
  recs[o] = r;
}

struct TopkShared {
  uint32_t keys[kTkCap];
  int list[kTkList];
  unsigned long long sel[kTkMaxK];
  unsigned long long sorted[kTkMaxK];
  int anchors[kTkMaxK];
  int over[kTkMaxK];
  int hist[256];
  unsigned long long diff;
  uint32_t smax;
  uint32_t wave_min[kTkThreads / 64], wave_max[kTkThreads / 64];
  int count, n_over;
  int digit, need, done;
};

static_assert(offsetof(TopkShared, sel) % 16 == 0, "rank counting reads two keys per 16-byte LDS access");

// Adds one to hist[dig] for every active lane of the wave.  The lanes sharing
// the first active lane's digit are counted by one atomic (in the early
// passes most keys share the top digits and would serialise on one LDS
// address); the other lanes add individually.
__device__ __forceinline__ void wave_histogram_add(int* hist, bool act, int dig) {
  const int lane = threadIdx.x & 63;
  const unsigned long long am = __ballot(act);
  if (am == 0) return;
  const int leader = __ffsll((long long)am) - 1;
  const int d = __shfl(dig, leader);
  const bool mine = act && dig == d;
  const unsigned long long same = __ballot(mine);
  if (lane == leader) atomicAdd(&hist[d], __popcll(same));
  if (act && !mine) atomicAdd(&hist[dig], 1);
}

// Slot of each lane with pred set in a compaction through *counter: one atomic
// per wave, lanes numbered in lane order.
__device__ __forceinline__ int wave_compact_slot(bool pred, int* counter) {
  const int lane = threadIdx.x & 63;
  const unsigned long long m = __ballot(pred);
  if (m == 0) return -1;
  const int leader = __ffsll((long long)m) - 1;
  int base = 0;
  if (lane == leader) base = atomicAdd(counter, __popcll(m));
  base = __shfl(base, leader);
  return pred ? base + __popcll(m & ((1ull << lane) - 1)) : -1;
}

// Stage-1 candidate i: full_key(keys[i], i) over the image's anchor keys in
// global memory (images with more anchors than the register chunks hold:
// every radix pass re-reads them from L2).
struct AllKeys {
  const uint32_t* keys;
  __device__ unsigned long long operator()(int i) const { return full_key(keys[i], (uint32_t)i); }
};
// Stage-2 tie index of class c of the j-th listed anchor (see the kernel).
struct TieIndex {
  const int* anchors;
  int nc;
  bool onnx;
  __device__ uint32_t operator()(int j, int c) const {
    return (uint32_t)(onnx ? j : anchors[j]) * (uint32_t)nc + (uint32_t)c;
  }
};
// Pair i = j * nc + c of the stage-2 key array (in LDS), keyed by its tie
// index.
struct TieKeys {
  const uint32_t* keys;
  TieIndex tie;
  __device__ unsigned long long operator()(int i) const {
    const int j = i / tie.nc;
    return full_key(keys[i], tie(j, i - j * tie.nc));
  }
};

// k-th largest of the n candidate keys get(i), i < n (1 <= k <= n).  Bits
// above the highest bit in which two candidates differ are shared by all of
// them and need no histogram pass; the 8-bit digit windows start below them
// (the last window may overlap bits already fixed, whose digits then agree
// with the prefix).
template <class Get>
__device__ unsigned long long radix_select(TopkShared& s, Get get, int n, int k) {
  const int lane = threadIdx.x & 63;
  const unsigned long long k0 = get(0);
  unsigned long long dv = 0;
  if (threadIdx.x == 0) s.diff = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) dv |= get(i) ^ k0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dv |= __shfl_xor(dv, off);
  if (lane == 0 && dv) atomicOr(&s.diff, dv);
  __syncthreads();
  const unsigned long long diff = s.diff;
  if (diff == 0) return k0;  // a single candidate
  const int top = 63 - __clzll((long long)diff);
  unsigned long long mask = top == 63 ? 0ull : ~0ull << (top + 1);
  unsigned long long prefix = k0 & mask;
  int need = k;
  for (int shift = top - 7;; shift -= 8) {
    if (shift < 0) shift = 0;
    for (int i = threadIdx.x; i < 256; i += blockDim.x) s.hist[i] = 0;
    __syncthreads();
    for (int base = 0; base < n; base += blockDim.x) {
      const int i = base + threadIdx.x;
      bool act = false;
      int dig = 0;
      if (i < n) {
        const unsigned long long key = get(i);
        act = (key & mask) == prefix;
        dig = (int)((key >> shift) & 255u);
      }
      wave_histogram_add(s.hist, act, dig);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      // Lane l holds bins 4l..4l+3.  S(d) = sum of bins >= d is non-increasing
      // in d; the digit is the largest d with S(d) >= need.
      const int h0 = s.hist[4 * lane], h1 = s.hist[4 * lane + 1], h2 = s.hist[4 * lane + 2],
                h3 = s.hist[4 * lane + 3];
      const int t = h0 + h1 + h2 + h3;
      int suf = t;  // inclusive suffix over lanes
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_down(suf, off);
        if (lane + off < 64) suf += y;
      }
      const int s3 = suf - t + h3, s2 = s3 + h2, s1 = s2 + h1, s0 = s1 + h0;
      int cnt = (s0 >= need) + (s1 >= need) + (s2 >= need) + (s3 >= need);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off);
      const int d = cnt - 1;
      if ((d >> 2) == lane) {
        const int j = d & 3;
        const int sd = j == 0 ? s0 : j == 1 ? s1 : j == 2 ? s2 : s3;
        const int hd = j == 0 ? h0 : j == 1 ? h1 : j == 2 ? h2 : h3;
        s.digit = d;
        s.need = need - (sd - hd);
        // Every key under the new prefix is selected: the prefix with zero
        // low bits is then a threshold with exactly k keys at or above it.
        s.done = hd == need - (sd - hd);
      }
    }
    __syncthreads();
    prefix |= (unsigned long long)s.digit << shift;
    mask |= 255ull << shift;
    need = s.need;
    if (s.done || shift == 0) break;
  }
  return prefix;
}

// Number of v[j0..j1) greater than key.  j0 is even and v 16-byte aligned,
// so two keys come per 16-byte LDS read, sixteen in flight per step.
__device__ __forceinline__ int count_greater(const unsigned long long* v, int j0, int j1, unsigned long long key) {
  int r = 0, j = j0;
  for (; j + 16 <= j1; j += 16) {
    ulonglong2 t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = *(const ulonglong2*)(v + j + 2 * u);
#pragma unroll
    for (int u = 0; u < 8; ++u) r += (t[u].x > key) + (t[u].y > key);
  }
  for (; j < j1; ++j) r += v[j] > key;
  return r;
}

// rank[i] = number of the k distinct keys s.sel[] greater than s.sel[i]
// (1 <= k <= blockDim.x).  Each key's count is split over blockDim.x / k
// threads; the ranks land in s.list (free outside the stage-2 compaction).
__device__ void rank_keys(TopkShared& s, int k) {
  for (int i = threadIdx.x; i < k; i += blockDim.x) s.list[i] = 0;
  __syncthreads();
  const int parts = blockDim.x / k, chunk = ((k + parts - 1) / parts + 1) & ~1;
  const int i = threadIdx.x % k, p = threadIdx.x / k;
  if (p < parts) {
    const int j0 = p * chunk, j1 = min(k, j0 + chunk);
    if (j0 < j1) atomicAdd(&s.list[i], count_greater(s.sel, j0, j1, s.sel[i]));
  }
  __syncthreads();
}

// The k keys >= threshold (exactly k: keys are unique), each placed at its
// rank, into s.sorted (descending).
template <class Get>
__device__ void collect_sorted(TopkShared& s, Get get, int n, int k, unsigned long long threshold) {
  if (threadIdx.x == 0) s.count = 0;
  __syncthreads();
  for (int base = 0; base < n; base += blockDim.x) {
    const int i = base + threadIdx.x;
    const unsigned long long key = i < n ? get(i) : 0ull;
    const bool take = i < n && key >= threshold;
    const int slot = wave_compact_slot(take, &s.count);
    if (take && slot < kTkMaxK) s.sel[slot] = key;
  }
  __syncthreads();
  rank_keys(s, k);
  for (int i = threadIdx.x; i < k; i += blockDim.x) s.sorted[s.list[i]] = s.sel[i];
  __syncthreads();
}

// ------------------------------------------------ stage 1 from registers
//
// For up to R * kTkThreads anchors the stage-1 keys stay in registers:
// thread t holds anchor c * kTkThreads + t as kr[c].  The radix select then
// reads no memory per pass and takes 11-bit digits (two passes usually
// isolate the k-th key).  Its histograms overlay the stage-2 key array,
// which is unused until stage 2.
constexpr int kTkWaves = kTkThreads / 64;
constexpr int kTkDigit = 11;
constexpr int kTkBins = 1 << kTkDigit;
// Bin d of a histogram sits at word d + 4 * (d / 32): the 32 bins each lane
// of the scanning wave reads start 36 words apart, so that wave's 16-byte
// reads spread over the LDS banks.
constexpr int kTkBinStride = kTkBins + kTkBins / 8;
constexpr int kTkMaxChunks = 33;  // register chunks of the largest instantiation

static_assert(2 * kTkBinStride + kTkMaxChunks * kTkWaves <= kTkCap, "stage-1 scratch overlays the key array");

__device__ __forceinline__ int bin_slot(int d) { return d + ((d >> 5) << 2); }

// Inclusive prefix over the lanes of a wave (every lane active), by DPP:
// Hillis-Steele steps inside each 16-lane row (row_shr 1, 2, 4, 8), then the
// row totals carried across rows (row_bcast 15 into rows 1 and 3, row_bcast
// 31 into rows 2 and 3).  A lane with no source lane reads 0, the identity of
// +, | and unsigned max.
template <int Ctrl, int Rows>
__device__ __forceinline__ int dpp_or_zero(int x) {
  return __builtin_amdgcn_update_dpp(0, x, Ctrl, Rows, 0xf, false);
}

template <class Op>
__device__ __forceinline__ int wave_prefix(int x, Op op) {
  x = op(x, dpp_or_zero<0x111, 0xf>(x));
  x = op(x, dpp_or_zero<0x112, 0xf>(x));
  x = op(x, dpp_or_zero<0x114, 0xf>(x));
  x = op(x, dpp_or_zero<0x118, 0xf>(x));
  x = op(x, dpp_or_zero<0x142, 0xa>(x));
  x = op(x, dpp_or_zero<0x143, 0xc>(x));
  return x;
}

__device__ __forceinline__ int wave_prefix_sum(int x) {
  return wave_prefix(x, [](int a, int b) { return a + b; });
}

// The unsigned maximum / minimum over the wave, in every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readlane(
      wave_prefix((int)x, [](int a, int b) { return (int)max((uint32_t)a, (uint32_t)b); }), 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) { return ~wave_max_u32(~x); }

// Run by one wave over an 11-bit histogram: the digit d of the k-th key
// under the current prefix (the largest d whose suffix count S(d), the keys in
// bins >= d, reaches need) and the count still needed inside bin d.  Lane l
// sums bin group 63 - l (bins 32g..32g+31 of group g), so the inclusive
// prefix over the lanes is S at each group's first bin and the first lane
// reaching need names the group holding d; lanes 0..31 then take that
// group's bins from the top and repeat the prefix over single bins.
__device__ __forceinline__ void digit_scan(TopkShared& s, const int* hist, int need) {
  const int lane = threadIdx.x & 63, g = 63 - lane;
  const int4* hv = reinterpret_cast<const int4*>(hist + 36 * g);
  int t = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int4 x = hv[q];
    t += (x.x + x.y) + (x.z + x.w);
  }
  // u grows over the lanes and the last lane's counts every key under the
  // prefix (at least need).
  const int u = wave_prefix_sum(t);
  const int first = __ffsll((long long)__ballot(u >= need)) - 1;
  const int gd = 63 - first;
  const int above = __builtin_amdgcn_readlane(u - t, first);  // keys in the groups above gd
  const int j = lane & 31;
  const int v = lane < 32 ? hist[36 * gd + 31 - j] : 0;  // bin 32 gd + 31 - j
  const int w = above + wave_prefix_sum(v);               // S(32 gd + 31 - j) on lanes 0..31
  const int hit = __ffsll((long long)__ballot(lane < 32 && w >= need)) - 1;
  if (lane == hit) {
    s.digit = 32 * gd + 31 - j;
    s.need = need - (w - v);
    s.done = v == need - (w - v);
  }
}

// k-th largest of the n register-held keys (1 <= k <= n), as radix_select
// with 11-bit digits, over v = key - (smallest score key << 32), so the
// first window spans the scores present rather than the float format: the
// scores' minimum and maximum give the top bit in which keys can differ (and
// every v is below 2^(top + 1), so the first pass counts every key).  kr is
// replaced by v and the threshold is returned in v's terms; `offset`
// receives the shift back to keys.  Each key under the prefix adds itself to
// its bin with one LDS atomic.
template <int R>
__device__ unsigned long long radix_select_regs(TopkShared& s, unsigned long long (&kr)[R], int n, int k,
                                                unsigned long long& offset) {
  int* H = reinterpret_cast<int*>(s.keys);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t lo = 0xffffffffu, hi = 0u;
#pragma unroll
  for (int c = 0; c < R; ++c) {
    if (c * kTkThreads + tid < n) {
      lo = min(lo, (uint32_t)(kr[c] >> 32));
      hi = max(hi, (uint32_t)(kr[c] >> 32));
    }
  }
  lo = wave_min_u32(lo);
  hi = wave_max_u32(hi);
  if (lane == 0) {
    s.wave_min[wave] = lo;
    s.wave_max[wave] = hi;
  }
  for (int i = tid; i < kTkBinStride; i += kTkThreads) H[i] = 0;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kTkWaves; ++w) {
    lo = min(lo, s.wave_min[w]);
    hi = max(hi, s.wave_max[w]);
  }
  offset = (unsigned long long)lo << 32;
  const uint32_t span = hi - lo;
#pragma unroll
  for (int c = 0; c < R; ++c) kr[c] -= offset;
  // All scores equal: the keys differ in the tie index only.
  const int top = span ? 63 - __clz((int)span) : 31;
  unsigned long long mask = top == 63 ? 0ull : ~0ull << (top + 1);
  unsigned long long prefix = 0;
  int need = k;
  for (int shift = top - (kTkDigit - 1), pass = 0;; shift -= kTkDigit, ++pass) {
    if (shift < 0) shift = 0;
    int* h = H + (pass & 1) * kTkBinStride;
    int* hn = H + ((pass + 1) & 1) * kTkBinStride;  // the next pass's histogram, scanned two passes ago
    for (int i = tid; i < kTkBinStride; i += kTkThreads) hn[i] = 0;
#pragma unroll
    for (int c = 0; c < R; ++c) {
      if (c * kTkThreads + tid < n && (pass == 0 || (kr[c] & mask) == prefix))
        atomicAdd(&h[bin_slot((int)((kr[c] >> shift) & (kTkBins - 1)))], 1);
    }
    __syncthreads();
    if (wave == 0) digit_scan(s, h, need);
    __syncthreads();
    prefix |= (unsigned long long)s.digit << shift;
    mask |= (unsigned long long)(kTkBins - 1) << shift;
    need = s.need;
    if (s.done || shift == 0) break;
  }
  return prefix;
}

// Exclusive prefix sums of v[0..n) in place, by one wave (lane l owns a run
// of ceil(n / 64) entries).
__device__ __forceinline__ void exclusive_scan_wave(int* v, int n) {
  const int lane = threadIdx.x & 63;
  const int per = (n + 63) >> 6, i0 = min(n, lane * per), i1 = min(n, i0 + per);
  int t = 0;
  for (int i = i0; i < i1; ++i) t += v[i];
  int run = wave_prefix_sum(t) - t;
  for (int i = i0; i < i1; ++i) {
    const int x = v[i];
    v[i] = run;
    run += x;
  }
}

// One wave's first slot in s.count for all lanes' hits of pred(0..N): one
// ballot per predicate, then one LDS atomic for the wave's total.  The
// caller numbers the hits in (predicate, lane) order from the result.
template <class Pred>
__device__ __forceinline__ int wave_reserve(TopkShared& s, int N, Pred pred) {
  int total = 0;
  for (int c = 0; c < N; ++c) total += __popcll(__ballot(pred(c)));
  int base = 0;
  if ((threadIdx.x & 63) == 0) base = atomicAdd(&s.count, total);
  return __builtin_amdgcn_readlane(base, 0);
}

// The k largest of the n listed stage-2 keys (k <= n <= kTkThreads, unique;
// thread t holds key t when `mine`) into s.sorted, descending: a counting
// sort on the top bits of each score above `bound` (256 buckets spanning the
// scores present, highest first), then each key's rank inside its bucket by
// direct comparison.  The caller has cleared s.hist and set s.smax to the
// largest listed score key, before a barrier.
__device__ void rank_listed(TopkShared& s, unsigned long long key, bool mine, int k, uint32_t bound) {
  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t spread = s.smax - bound;
  const int sh = spread < 256u ? 0 : 24 - __clz((int)spread);  // (spread >> sh) < 256
  const int bucket = mine ? (int)(((uint32_t)(key >> 32) - bound) >> sh) : 0;
  int pos = 0;
  if (mine) pos = atomicAdd(&s.hist[bucket], 1);
  __syncthreads();
  int* start = s.over;  // bucket starts; s.hist keeps the counts
  if (tid < 64) {
    int c[4], t = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c[q] = s.hist[255 - 4 * lane - q];
      t += c[q];
    }
    int run = wave_prefix_sum(t) - t;  // keys in buckets above this lane's
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      start[255 - 4 * lane - q] = run;
      run += c[q];
    }
  }
  __syncthreads();
  unsigned long long* grouped = s.sel;  // keys by bucket (every key is in a register now)
  const int b0 = start[bucket], nb = s.hist[bucket];
  if (mine) grouped[b0 + pos] = key;
  __syncthreads();
  if (mine) {
    int r = b0;
    for (int j = b0; j < b0 + nb; ++j) r += grouped[j] > key;
    if (r < k) s.sorted[r] = key;
  }
  __syncthreads();
}

// Stage 1 over register-held keys (n <= R * kTkThreads): s.anchors[0..k) in
// stage-2 enumeration order; returns the stage-1 threshold (exactly k keys
// are at or above it).
template <int R>
__device__ unsigned long long stage1_registers(TopkShared& s, const uint32_t* __restrict__ kb, int n, int k, bool ox) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int* H = reinterpret_cast<int*>(s.keys);
  unsigned long long kr[R];
#pragma unroll
  for (int c = 0; c < R; ++c) {
    const int a = c * kTkThreads + tid;
    kr[c] = a < n ? full_key(kb[a], (uint32_t)a) : 0ull;
  }
  if (tid == 0) {
    s.smax = 0u;
    s.count = 0;
  }
  unsigned long long offset;
  const unsigned long long tv = radix_select_regs<R>(s, kr, n, k, offset);  // kr now holds key - offset
  const unsigned long long t1 = tv + offset;
  if (!ox) {
    // Under PT rules stage 2 ties by anchor index (tie index anchor * nc +
    // class), so the selected anchors may be listed in any order.
    int run = wave_reserve(s, R, [&](int c) { return c * kTkThreads + tid < n && kr[c] >= tv; });
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int c = 0; c < R; ++c) {
      const bool take = c * kTkThreads + tid < n && kr[c] >= tv;
      const unsigned long long m = __ballot(take);
      if (take) s.anchors[run + __popcll(m & below)] = c * kTkThreads + tid;
      run += __popcll(m);
    }
  } else {
    // ONNX rules: the k keys >= t1 collected in any order, then ranked
    // among themselves (one per thread).
    int run = wave_reserve(s, R, [&](int c) { return c * kTkThreads + tid < n && kr[c] >= tv; });
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int c = 0; c < R; ++c) {
      const bool take = c * kTkThreads + tid < n && kr[c] >= tv;
      const unsigned long long m = __ballot(take);
      if (take) s.sel[run + __popcll(m & below)] = kr[c] + offset;
      run += __popcll(m);
    }
    if (tid < 256) s.hist[tid] = 0;
    __syncthreads();
    const bool mine = tid < k;
    const unsigned long long key = mine ? s.sel[tid] : 0ull;
    const uint32_t wmax = wave_max_u32((uint32_t)(key >> 32));
    if (lane == 0) atomicMax(&s.smax, wmax);
    __syncthreads();
    rank_listed(s, key, mine, k, (uint32_t)(t1 >> 32));
    for (int i = tid; i < k; i += kTkThreads) s.anchors[i] = (int)(0xffffffffu - (uint32_t)s.sorted[i]);
  }
  __syncthreads();
  return t1;
}

// Stage 1 over keys read from global memory on every pass (images with more
// anchors than the register chunks hold).
__device__ unsigned long long stage1_global(TopkShared& s, const uint32_t* __restrict__ kb, int n, int k, bool ox) {
  const AllKeys stage1{kb};
  const unsigned long long t1 = radix_select(s, stage1, n, k);
  if (ox) {
    collect_sorted(s, stage1, n, k, t1);
    for (int i = threadIdx.x; i < k; i += blockDim.x) s.anchors[i] = (int)(0xffffffffu - (uint32_t)s.sorted[i]);
  } else {
    // An order-preserving compaction: thread t owns a contiguous run of
    // anchors, counts its selected ones, and writes them at its exclusive
    // prefix over the workgroup.
    const int per = (n + kTkThreads - 1) / kTkThreads;
    const int a0 = min(n, (int)threadIdx.x * per), a1 = min(n, a0 + per);
    int cnt = 0;
    for (int a = a0; a < a1; ++a) cnt += stage1(a) >= t1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = cnt;  // inclusive scan within the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(inc, off);
      if (lane >= off) inc += y;
    }
    if (lane == 63) s.hist[wave] = inc;
    __syncthreads();
    int woff = 0;
    for (int w = 0; w < wave; ++w) woff += s.hist[w];
    int slot = woff + inc - cnt;
    for (int a = a0; a < a1; ++a)
      if (stage1(a) >= t1) s.anchors[slot++] = a;
  }
  __syncthreads();
  return t1;
}

// One image per workgroup: stage 1 (R > 0: keys in R register chunks;
// R == 0: keys from global memory), stage 2, and the first six fields of the
// image's output rows (x, y, w/x2, h/y2, score, class as float); with extra
// fields, the picks (anchor, class) for topk_extras_kernel.
template <int R>
__global__ __launch_bounds__(kTkThreads) void topk_select_kernel(const float* __restrict__ head,
                                                                const uint32_t* __restrict__ keys1,
                                                                const TopRec* __restrict__ recs, int channels,
                                                                int anchors, int nc, int k, int onnx,
                                                                float* __restrict__ out, int2* __restrict__ picks) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  TopkShared& s = *reinterpret_cast<TopkShared*>(smem);
  const int b = blockIdx.x;
  const float* src = head + (long long)b * channels * anchors;
  const bool ox = onnx != 0;
  const uint32_t* kb = keys1 + (long long)b * anchors;
  unsigned long long t1;
  if constexpr (R > 0) {
    t1 = stage1_registers<R>(s, kb, anchors, k, ox);
  } else {
    t1 = stage1_global(s, kb, anchors, k, ox);
  }
  const uint32_t bound = (uint32_t)(t1 >> 32);
  if (threadIdx.x == 0) {
    s.count = 0;
    s.n_over = 0;
    s.smax = 0;
  }
  __syncthreads();
  // Stage 2 candidates at or above the bound, from the four-best records:
  // each listed record whose truncated key reaches the bound's has its exact
  // score re-read (the loads of a thread's four records issued before their
  // use), and goes to the rank list as a full key.  An anchor whose fourth
  // record reaches the bound's truncated key may have more: its whole column
  // is read below.  The tie index of class c of the j-th listed anchor is
  // tie(j, c): j * nc + c under ONNX rules (the list is in stage-1 rank
  // order), anchor * nc + c under PT rules.
  const TopRec* rb = recs + (long long)b * anchors;
  const uint32_t tb = bound >> 7;
  const TieIndex tie{s.anchors, nc, ox};
  for (int base = 0; base < k; base += kTkThreads) {
    const int j = base + threadIdx.x;
    const int a = s.anchors[min(j, k - 1)];
    const TopRec r = rb[a];
    const bool over = j < k && nc > kTkRec && (nc > kTkRecClasses || (r.r[kTkRec - 1] >> 7) >= tb);
    bool cand[kTkRec];
    int cls[kTkRec];
    float v[kTkRec];
#pragma unroll
    for (int p = 0; p < kTkRec; ++p) {
      cand[p] = j < k && !over && r.r[p] != 0u && (r.r[p] >> 7) >= tb;
      cls[p] = cand[p] ? min(127 - (int)(r.r[p] & 127u), nc - 1) : 0;  // a record's class is below nc
      v[p] = src[(long long)(4 + cls[p]) * anchors + a];
    }
    // Slots for the wave's kept records and over-anchors: one ballot each,
    // one atomic per counter.
    uint32_t key[kTkRec];
    bool keep[kTkRec];
    int total = 0;
#pragma unroll
    for (int p = 0; p < kTkRec; ++p) {
      key[p] = score_key(v[p], ox);
      keep[p] = cand[p] && key[p] >= bound;
      total += __popcll(__ballot(keep[p]));
    }
    const unsigned long long om = __ballot(over);
    int run = 0, obase = 0;
    if ((threadIdx.x & 63) == 0) {
      run = atomicAdd(&s.count, total);
      obase = om ? atomicAdd(&s.n_over, __popcll(om)) : 0;
    }
    run = __builtin_amdgcn_readlane(run, 0);
    obase = __builtin_amdgcn_readlane(obase, 0);
    const unsigned long long below = (1ull << (threadIdx.x & 63)) - 1ull;
    if (over) s.over[obase + __popcll(om & below)] = j;
#pragma unroll
    for (int p = 0; p < kTkRec; ++p) {
      const unsigned long long m = __ballot(keep[p]);
      const int slot = run + __popcll(m & below);
      if (keep[p] && slot < kTkList) s.sel[slot] = full_key(key[p], tie(j, cls[p]));
      run += __popcll(m);
    }
  }
  __syncthreads();
  const int n_over = s.n_over, n2 = k * nc;
  for (int base = 0; base < n_over * nc; base += 4 * kTkThreads) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = min(base + u * kTkThreads + (int)threadIdx.x, n_over * nc - 1);
      const int j = s.over[t / nc], c = t - (t / nc) * nc;
      v[u] = src[(long long)(4 + c) * anchors + s.anchors[j]];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = base + u * kTkThreads + (int)threadIdx.x;
      const bool in = t < n_over * nc;
      const int j = in ? s.over[t / nc] : 0, c = t - (t / nc) * nc;
      const uint32_t key = in ? score_key(v[u], ox) : 0u;
      const bool keep = in && key >= bound;
      const int slot = wave_compact_slot(keep, &s.count);
      if (keep && slot < kTkList) s.sel[slot] = full_key(key, tie(j, c));
    }
  }
  __syncthreads();
  const int listed = s.count;
  __syncthreads();
  if (listed <= kTkList) {
    // The listed keys (at least k), one per thread, ranked among themselves.
    const int tid = threadIdx.x;
    const bool mine = tid < listed;
    const unsigned long long key = mine ? s.sel[tid] : 0ull;
    if (tid < 256) s.hist[tid] = 0;
    const uint32_t wmax = wave_max_u32((uint32_t)(key >> 32));
    if ((tid & 63) == 0) atomicMax(&s.smax, wmax);
    __syncthreads();
    rank_listed(s, key, mine, k, bound);
  } else {
    // A flood of ties at the bound: every pair's key, then the full select.
    const TieKeys all{s.keys, tie};
    constexpr int U = 8;
    for (int base = 0; base < n2; base += U * kTkThreads) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = base + u * kTkThreads + threadIdx.x;
        v[u] = 0.f;
        if (e < n2) {
          const int j = e / nc, c = e - (e / nc) * nc;
          v[u] = src[(long long)(4 + c) * anchors + s.anchors[j]];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = base + u * kTkThreads + threadIdx.x;
        if (e < n2) s.keys[e] = score_key(v[u], ox);
      }
    }
    __syncthreads();
    collect_sorted(s, all, n2, k, radix_select(s, all, n2, k));
  }
  // The picks (anchor, class) of rows 0..k), then the rows themselves, eight
  // gathers in flight per thread.
  int* pick_anchor = s.list;
  int* pick_class = s.over;
  for (int i = threadIdx.x; i < k; i += kTkThreads) {
    const uint32_t e = 0xffffffffu - (uint32_t)s.sorted[i];
    const int q = (int)(e / (uint32_t)nc);
    pick_anchor[i] = ox ? s.anchors[min(q, k - 1)] : min(q, anchors - 1);
    pick_class[i] = min((int)(e - (uint32_t)q * (uint32_t)nc), nc - 1);
  }
  __syncthreads();
  // The rows' first six fields; the extra fields (mask coefficients,
  // keypoints) are scattered gathers, left to topk_extras_kernel over the
  // whole GPU, which reads the picks.
  const int fields = channels - nc + 2, total = k * 6;
  float* ob = out + (long long)b * k * fields;
  if (picks)
    for (int i = threadIdx.x; i < k; i += kTkThreads) picks[(long long)b * k + i] = int2{pick_anchor[i], pick_class[i]};
  constexpr int U = 8;
  for (int base = 0; base < total; base += U * kTkThreads) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = base + u * kTkThreads + (int)threadIdx.x;
      v[u] = 0.f;
      if (idx < total) {
        const int i = idx / 6, f = idx - (idx / 6) * 6;
        const int a = pick_anchor[i], c = pick_class[i];
        if (f == 5) v[u] = (float)c;
        else v[u] = src[(long long)(f < 4 ? f : 4 + c) * anchors + a];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = base + u * kTkThreads + (int)threadIdx.x;
      if (idx < total) {
        const int i = idx / 6;
        ob[(long long)i * fields + (idx - i * 6)] = v[u];
      }
    }
  }
}

// Fields 6.. of each output row (the head's channels after the classes) for
// the picks (anchor, class) of image blockIdx.y.
__global__ __launch_bounds__(256) void topk_extras_kernel(const float* __restrict__ head, const int2* __restrict__ picks,
                                                          int channels, int anchors, int nc, int k,
                                                          float* __restrict__ out) {
  const int b = blockIdx.y;
  const int extra = channels - nc - 4, fields = extra + 6;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= k * extra) return;
  const int i = idx / extra, f = idx - (idx / extra) * extra;
  const int a = picks[(long long)b * k + i].x;
  out[((long long)b * k + i) * fields + 6 + f] = head[((long long)b * channels + nc + 4 + f) * anchors + a];
}

// Arguments of a top-k call, checked once for both entry points.
struct TopkCall {
  const float* head;
  int batch, channels, anchors, nc, k, onnx, fields;
  float* out;
  size_t keys_b, recs_b, picks_b;  // scratch layout: stage-1 keys, four-best lists, picks
};

static int topk_check(const float* head, int batch, int channels, int anchors, int nc, int maximum, int onnx,
                      float* out, TopkCall* c) {
  SY_CHECK(head && out, SY_EINVAL, "null argument");
  SY_CHECK(batch >= 0 && anchors >= 0 && nc > 0 && channels >= nc + 4 && maximum >= 0, SY_EINVAL,
           "invalid top-k arguments");
  SY_CHECK(!onnx || maximum <= anchors, SY_EINVAL, "ONNX rules need maximum <= anchors");
  const int k = maximum < anchors ? maximum : anchors;
  *c = TopkCall{head, batch, channels, anchors, nc, k, onnx ? 1 : 0, channels - nc + 2, out, 0, 0, 0};
  if (batch == 0 || k == 0) return SY_OK;
  SY_CHECK(k <= kTkMaxK, SY_EUNSUPPORTED, "top-k of %d exceeds %d", k, kTkMaxK);
  SY_CHECK(anchors <= kTkMaxAnchors && (long long)k * nc <= kTkCap, SY_EUNSUPPORTED,
           "top-k of %d over %d anchors x %d classes exceeds the limits (%d anchors, k x classes %d)", k, anchors, nc,
           kTkMaxAnchors, kTkCap);
  SY_CHECK(batch <= 65535, SY_EUNSUPPORTED, "top-k batch too large");
  SY_CHECK((long long)anchors * nc < 0xffffffffLL, SY_EUNSUPPORTED,
           "top-k of %d anchors x %d classes: the pair tie index exceeds 32 bits", anchors, nc);
  SY_CHECK((long long)k * c->fields <= 0x7fffffffLL - 255, SY_EUNSUPPORTED, "top-k output too large");
  auto align = [](size_t v) { return (v + 255) & ~size_t(255); };
  c->keys_b = align((size_t)batch * anchors * sizeof(uint32_t));
  c->recs_b = align((size_t)batch * anchors * sizeof(TopRec));
  c->picks_b = c->fields > 6 ? align((size_t)batch * k * sizeof(int2)) : 0;
  return SY_OK;
}

int e2e_topk_scratch_bytes(int batch, int channels, int anchors, int nc, int maximum, size_t* bytes) {
  TopkCall c;
  float probe = 0.f;
  SY_TRY(topk_check(&probe, batch, channels, anchors, nc, maximum, 0, &probe, &c));
  *bytes = c.keys_b + c.recs_b + c.picks_b;
  return SY_OK;
}

// Register chunks of stage-1 keys per thread for an image of `anchors`
// (0: more than the largest instantiation holds; the keys are read from
// global memory on every pass).
static int select_chunks(int anchors) {
  const int chunks = (anchors + kTkThreads - 1) / kTkThreads;
  return chunks <= 3 ? 3 : chunks <= 9 ? 9 : chunks <= 17 ? 17 : chunks <= kTkMaxChunks ? kTkMaxChunks : 0;
}

template <int R>
static void launch_select(const TopkCall& c, const uint32_t* keys1, const TopRec* recs, int2* picks,
                          hipStream_t stream) {
  hipLaunchKernelGGL(topk_select_kernel<R>, dim3(c.batch), dim3(kTkThreads), sizeof(TopkShared), stream, c.head,
                     keys1, recs, c.channels, c.anchors, c.nc, c.k, c.onnx, c.out, picks);
}

// The kernels on ctx->stream over a scratch block of at least
// keys_b + recs_b + picks_b bytes.  Every scratch byte a kernel reads was written
// earlier in the same call, so the block needs no clearing.
static int topk_launch(sy_ctx* ctx, const TopkCall& c, char* base, bool profile) {
  uint32_t* keys1 = (uint32_t*)base;
  TopRec* recs = (TopRec*)(base + c.keys_b);
  int2* picks = c.picks_b ? (int2*)(base + c.keys_b + c.recs_b) : nullptr;
  sy_ctx* pc = profile ? ctx : nullptr;
  const double score_bytes = 4.0 * (double)c.batch * c.anchors * c.nc;
  {
    ProfScope prof(pc, "topk_class_pass", 0, score_bytes + (4.0 + sizeof(TopRec)) * c.batch * c.anchors);
    const dim3 grid((unsigned)((c.anchors + kTkGroup - 1) / kTkGroup), (unsigned)c.batch);
    hipLaunchKernelGGL(topk_class_pass_kernel, grid, dim3(256), 0, ctx->stream, c.head, c.channels, c.anchors,
                       c.nc, c.onnx, keys1, recs);
    SY_TRY(check_launch("topk_class_pass"));
  }
  {
    // The select kernels' LDS limit is raised in topk_static_init.
    ProfScope prof(pc, "topk_select", 0,
                   (double)c.batch * (4.0 * c.anchors + (double)c.k * (sizeof(TopRec) + 8.0 + 48.0)));
    switch (select_chunks(c.anchors)) {
      case 3: launch_select<3>(c, keys1, recs, picks, ctx->stream); break;
      case 9: launch_select<9>(c, keys1, recs, picks, ctx->stream); break;
      case 17: launch_select<17>(c, keys1, recs, picks, ctx->stream); break;
      case kTkMaxChunks: launch_select<kTkMaxChunks>(c, keys1, recs, picks, ctx->stream); break;
      default: launch_select<0>(c, keys1, recs, picks, ctx->stream); break;
    }
    SY_TRY(check_launch("topk_select"));
  }
  if (!picks) return SY_OK;
  const int extra = c.fields - 6;
  ProfScope prof(pc, "topk_extras", 0, (double)c.batch * c.k * (8.0 + 8.0 * extra));
  const dim3 grid((unsigned)((c.k * extra + 255) / 256), (unsigned)c.batch);
  hipLaunchKernelGGL(topk_extras_kernel, grid, dim3(256), 0, ctx->stream, c.head, picks, c.channels, c.anchors, c.nc,
                     c.k, c.out);
  return check_launch("topk_extras");
}

int op_e2e_topk(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum, int onnx,
                float* out) {
  TopkCall c;
  SY_TRY(topk_check(head, batch, channels, anchors, nc, maximum, onnx, out, &c));
  if (batch == 0 || c.k == 0) return SY_OK;
  SY_TRY(ensure_scratch(ctx, c.keys_b + c.recs_b + c.picks_b));
  return topk_launch(ctx, c, ctx->scratch, true);
}

// ------------------------------------------------- allocation-free variant
//
// Callers that may not allocate device memory (graph capture, serving loops)
// use a fixed block in the code object instead of the context scratch: one
// copy per GPU, held until the process ends.  In host code `scratch` only
// names the symbol; its device address is looked up per device with that
// device current (topk_static_init, from sy_create) and used everywhere.
// Calls on one GPU share the block, so calls that overlap in time on that GPU
// (two contexts, two streams) race on it.
static __device__ __align__(256) unsigned char scratch[kTopkStaticScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_static_mu;
static char* g_static_ptr[kMaxDevices];
// Per device: the event recorded after the last allocation-free call's
// kernels, which the next call's stream waits on (calls from different
// contexts or streams are ordered on the block instead of racing on it).
static hipEvent_t g_static_done[kMaxDevices];
static bool g_static_recorded[kMaxDevices];

// Called by sy_create with `device` current: the select kernels' LDS limit
// (process-wide), the block's device address and the ordering event.
int topk_static_init(int device) {
  SY_CHECK(device >= 0 && device < kMaxDevices, SY_EUNSUPPORTED, "device %d beyond the %d the library tracks", device,
           kMaxDevices);
  std::lock_guard<std::mutex> lock(g_static_mu);
  if (g_static_ptr[device]) return SY_OK;
  const void* selects[] = {(const void*)topk_select_kernel<3>, (const void*)topk_select_kernel<9>,
                           (const void*)topk_select_kernel<17>, (const void*)topk_select_kernel<kTkMaxChunks>,
                           (const void*)topk_select_kernel<0>};
  for (const void* fn : selects)
    SY_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(TopkShared)));
  void* ptr = nullptr;
  SY_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  SY_CHECK(ptr != nullptr, SY_EDEVICE, "no device address for the static top-k scratch");
  SY_HIP(hipEventCreateWithFlags(&g_static_done[device], hipEventDisableTiming));
  g_static_ptr[device] = (char*)ptr;
  return SY_OK;
}

int op_e2e_topk_noalloc(sy_ctx* ctx, const float* head, int batch, int channels, int anchors, int nc, int maximum,
                        int onnx, float* out) {
  TopkCall c;
  SY_TRY(topk_check(head, batch, channels, anchors, nc, maximum, onnx, out, &c));
  if (batch == 0 || c.k == 0) return SY_OK;
  const size_t need = c.keys_b + c.recs_b + c.picks_b;
  SY_CHECK(need <= kTopkStaticScratchBytes, SY_EUNSUPPORTED,
           "allocation-free top-k needs %zu bytes of scratch for batch %d x %d anchors (k = %d); its fixed block "
           "holds %zu (about %zu anchor-images)",
           need, batch, anchors, c.k, kTopkStaticScratchBytes,
           kTopkStaticScratchBytes / (sizeof(uint32_t) + sizeof(TopRec)));
  const int dev = ctx->device;
  SY_CHECK(dev >= 0 && dev < kMaxDevices, SY_ESTATE, "device %d has no static top-k scratch", dev);
  // The lock spans the wait, the launches and the record, so the calls on a
  // device enqueue in one order and each one's kernels start after the
  // previous one's finished.  Under graph capture the wait and record are
  // not recorded (an event from outside a capture cannot be waited on inside
  // it): the caller orders the graph's launches against other calls.
  std::lock_guard<std::mutex> lock(g_static_mu);
  char* base = g_static_ptr[dev];
  SY_CHECK(base != nullptr, SY_ESTATE, "static top-k scratch of device %d was not initialised", dev);
  if (!ctx->capturing && g_static_recorded[dev]) SY_HIP(hipStreamWaitEvent(ctx->stream, g_static_done[dev], 0));
  SY_TRY(topk_launch(ctx, c, base, false));
  if (!ctx->capturing) {
    SY_HIP(hipEventRecord(g_static_done[dev], ctx->stream));
    g_static_recorded[dev] = true;
  }
  return SY_OK;
}

}  // namespace sy
