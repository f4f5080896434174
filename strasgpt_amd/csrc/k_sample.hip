// Stochastic token sampling on the device: the steps of the reference's
// sampler_sample (source/sampler.c:234-337) on logits already in HBM.
//
//   presence penalty (source/sampler.c:238-248): logits of tokens seen
//     (the previous token is marked first) lower by the penalty;
//   greedy (temperature 0): the first index of the maximum (argmax kernels);
//   else: logits / temperature, softmax (max, expf(x - max), divide by the
//     sum), one xorshift64* coin, top-k (the k most likely), top-p (the
//     shortest descending prefix whose running sum reaches top_p),
//     renormalisation (double sum), and the first index whose running sum
//     of probabilities in index order exceeds the coin.
//
// Differences from the sequential host code are in summation order only:
// the softmax sum, the top-p running sum and the index-order running sum
// are formed from fixed-order partial sums (deterministic, but rounded
// differently), so a draw can differ from the reference's only when the
// coin or top_p lies within that rounding of a boundary. Equal
// probabilities rank by index (the radix sort below is stable), as a
// stable sort of the reference's index-ordered array ranks them. The coin stream, the
// penalty and every per-element operation (division by the temperature,
// expf, division by the sum, multiplication by the float inverse of the
// double sum) are the reference's.
#include <limits.h>

#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {
namespace {

constexpr int kSB = 256;    // blocks of the element-wise passes
constexpr int kST = 256;    // their threads
constexpr int kPick = 1024; // threads of the single-block passes
static_assert(kSB == kST, "the per-block partials are reduced by one block of kST threads");

__device__ __forceinline__ float block_max256(float v, float* red) {
  v = wave_peak(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kST / WAVE; i++) m = fmaxf(m, red[i]);
  __syncthreads();
  return m;
}

// Penalty, temperature, per-block maxima. Marks the previous token present.
__global__ __launch_bounds__(kST) void sample_scale_kernel(SampleParams p) {
  __shared__ float red[kST / WAVE];
  const int prev = p.prev ? *p.prev : p.prev_value;
  float m = -INFINITY;
  for (int i = blockIdx.x * kST + threadIdx.x; i < p.V; i += kSB * kST) {
    float x = p.logits[i];
    if (p.penalty != 0.0f && (p.presence[i] || i == prev)) x -= p.penalty;
    if (p.temperature != 0.0f) x = x / p.temperature;
    p.y[i] = x;
    m = fmaxf(m, x);
  }
  m = block_max256(m, red);
  if (threadIdx.x == 0) p.part[blockIdx.x] = m;
  if (blockIdx.x == 0 && threadIdx.x == 0 && prev >= 0 && prev < p.V) p.presence[prev] = 1;
}

// expf(x - max) in place, per-block sums.
__global__ __launch_bounds__(kST) void sample_exp_kernel(SampleParams p) {
  __shared__ float red[kST / WAVE];
  const float mx = block_max256(p.part[threadIdx.x], red);  // the same in every block
  float s = 0.0f;
  for (int i = blockIdx.x * kST + threadIdx.x; i < p.V; i += kSB * kST) {
    const float e = expf(p.y[i] - mx);
    p.y[i] = e;
    s += e;
  }
  s = block_sum<kST>(s, red);
  if (threadIdx.x == 0) p.part[kSB + blockIdx.x] = s;
}

// Probabilities, the sort keys, cleared keep marks, and the coin.
__global__ __launch_bounds__(kST) void sample_norm_kernel(SampleParams p) {
  __shared__ float red[kST / WAVE];
  const float sum = block_sum<kST>(p.part[kSB + threadIdx.x], red);  // the same in every block
  for (int i = blockIdx.x * kST + threadIdx.x; i < p.V; i += kSB * kST) {
    const float q = p.y[i] / sum;
    p.y[i] = q;
    if (p.keys) {
      p.keys[i] = __float_as_uint(q);  // q >= 0: the bit patterns order like the values
      p.vals[i] = i;
      p.keep[i] = 0;
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    unsigned long long s = *p.rng;  // xorshift64* (source/sampler.c:79-90)
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *p.rng = s;
    const unsigned u = (unsigned)((s * 0x2545F4914F6CDD1Dull) >> 32);
    p.scal[0] = (float)(u >> 8) / 16777216.0f;
  }
}

__device__ __forceinline__ double block_sum_d(double v, double* red) {
  red[threadIdx.x] = v;
  __syncthreads();
  for (int st = kPick / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
    __syncthreads();
  }
  const double s = red[0];
  __syncthreads();
  return s;
}

// Top-k / top-p cut over the descending order, the renormalisation factor,
// and the kept tokens' marks.
__global__ __launch_bounds__(kPick) void sample_select_kernel(SampleParams p) {
  __shared__ float scan[2][kPick];
  __shared__ double dred[kPick];
  __shared__ int found;
  const int tid = threadIdx.x, V = p.V;
  const bool sorted = p.keys != nullptr;
  int n = V;
  if (sorted) {
    const int kact = p.top_k > 0 && p.top_k < V ? p.top_k : V;
    n = kact;
    if (p.top_p > 0.0f && p.top_p <= 1.0f) {
      if (tid == 0) found = INT_MAX;
      float carry = 0.0f;
      __syncthreads();
      for (int base = 0; base < kact; base += kPick) {
        const int i = base + tid;
        float v = i < kact ? __uint_as_float(p.keys_sorted[i]) : 0.0f;
        int cur = 0;
        scan[0][tid] = v;
        __syncthreads();
        for (int off = 1; off < kPick; off <<= 1) {  // inclusive scan, fixed order
          const float add = tid >= off ? scan[cur][tid - off] : 0.0f;
          scan[cur ^ 1][tid] = scan[cur][tid] + add;
          cur ^= 1;
          __syncthreads();
        }
        const float cum = carry + scan[cur][tid];
        if (i < kact && cum >= p.top_p) atomicMin(&found, i);  // the first index reaching top_p
        __syncthreads();
        carry += scan[cur][kPick - 1];
        __syncthreads();
        if (found != INT_MAX) break;
      }
      if (found != INT_MAX) n = found + 1 < kact ? found + 1 : kact;
    }
  }
  double s = 0.0;
  if (sorted) {
    for (int r = tid; r < n; r += kPick) s += (double)__uint_as_float(p.keys_sorted[r]);
  } else {
    for (int i = tid; i < V; i += kPick) s += (double)p.y[i];
  }
  s = block_sum_d(s, dred);
  if (sorted)
    for (int r = tid; r < n; r += kPick) p.keep[p.vals_sorted[r]] = 1;
  if (tid == 0) {
    p.scal[1] = s > 0.0 ? (float)(1.0 / s) : 0.0f;
    p.scal[2] = s > 0.0 ? 0.0f : 1.0f;  // nothing left: uniform over every token
    *p.nkeep = n;
  }
}

// The first index of nonzero weight whose running sum of renormalised
// probabilities (index order) exceeds the coin; then the token bookkeeping
// of the decode loop.
__global__ __launch_bounds__(kPick) void sample_pick_kernel(SampleParams p) {
  __shared__ float pre[kPick];
  __shared__ int best;
  const int tid = threadIdx.x, V = p.V;
  const float coin = p.scal[0], inv = p.scal[1];
  const bool uniform = p.scal[2] != 0.0f, all = p.keys == nullptr;
  const float u = 1.0f / (float)V;
  const int R = (V + kPick - 1) / kPick, lo = min(V, tid * R), hi = min(V, lo + R);
  auto w = [&](int i) -> float {
    return uniform ? u : (all || p.keep[i]) ? p.y[i] * inv : 0.0f;
  };
  float s = 0.0f;
  for (int i = lo; i < hi; i++) s += w(i);
  pre[tid] = s;
  if (tid == 0) best = V;
  __syncthreads();
  if (tid == 0) {  // exclusive prefix in thread order, sequential
    float c = 0.0f;
    for (int t = 0; t < kPick; t++) {
      const float x = pre[t];
      pre[t] = c;
      c += x;
    }
  }
  __syncthreads();
  // A thread's start (the prefix of separately summed partials) can round
  // above the previous thread's last running sum; only an index of nonzero
  // weight is taken, so a coin in that gap never picks a token that top-k or
  // top-p removed (the reference's loop never returns one either).
  float cdf = pre[tid];
  for (int i = lo; i < hi; i++) {
    const float wi = w(i);
    cdf += wi;
    if (wi > 0.0f && coin < cdf) {
      atomicMin(&best, i);
      break;
    }
  }
  __syncthreads();
  if (tid == 0) {
    const int tok = best < V ? best : V - 1;  // rounding fallback, as the reference's
    *p.out = tok;
    if (p.seq) p.seq[(*p.seq_len)++] = tok;
    if (p.pos_inc) (*p.pos_inc)++;
  }
}

// ------------------------------------------------------------ radix sort --
// Stable descending sort of (key, value) pairs: a least-significant-digit
// radix sort of the inverted keys (ascending on ~key is descending on key),
// four passes of 8-bit digits. A pass is three launches over kRsBlocks
// contiguous chunks of the input:
// * histogram: the digit counts of each chunk, stored bin-major
//   (hist[digit][chunk]);
// * scan: one block turns them into exclusive offsets in that order, so a
//   digit's elements of chunk c land after those of chunks < c;
// * scatter: each chunk, in tiles of kRsThreads elements in input order,
//   ranks every element among the equal digits of its tile (within a
//   wavefront by ballots over the digit's bits, across wavefronts by
//   per-wavefront counts) and writes it at its digit's running offset.
// Every step keeps input order among equal digits, hence the stability.
constexpr int kRsThreads = 256;
constexpr int kRsWaves = kRsThreads / WAVE;
constexpr int kRsBlocks = 64;
constexpr int kRsBins = 256;
constexpr int kRsScan = 1024;  // threads of the scan: kRsBins * kRsBlocks / kRsScan entries each
static_assert(kRsBins * kRsBlocks % kRsScan == 0, "scan partition");

__device__ __forceinline__ int rs_chunk(int n) { return (n + kRsBlocks - 1) / kRsBlocks; }
__device__ __forceinline__ unsigned rs_digit(unsigned key, int shift) { return (~key >> shift) & (kRsBins - 1); }

__global__ __launch_bounds__(kRsThreads) void rs_hist_kernel(const unsigned* keys, int n, int shift,
                                                           unsigned* hist) {
  __shared__ unsigned h[kRsBins];
  for (int i = threadIdx.x; i < kRsBins; i += kRsThreads) h[i] = 0u;
  __syncthreads();
  const int ch = rs_chunk(n), lo = min(n, (int)blockIdx.x * ch), hi = min(n, lo + ch);
  for (int i = lo + threadIdx.x; i < hi; i += kRsThreads) atomicAdd(&h[rs_digit(keys[i], shift)], 1u);
  __syncthreads();
  for (int d = threadIdx.x; d < kRsBins; d += kRsThreads) hist[d * kRsBlocks + blockIdx.x] = h[d];
}

// Exclusive scan of the kRsBins * kRsBlocks counts in place: each thread a
// run of consecutive entries, then a scan of the runs' sums in thread order.
__global__ __launch_bounds__(kRsScan) void rs_scan_kernel(unsigned* hist) {
  constexpr int PER = kRsBins * kRsBlocks / kRsScan;
  __shared__ unsigned run[2][kRsScan];
  const int t = threadIdx.x;
  unsigned v[PER], sum = 0u;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    v[i] = hist[t * PER + i];
    sum += v[i];
  }
  int cur = 0;
  run[0][t] = sum;
  __syncthreads();
  for (int off = 1; off < kRsScan; off <<= 1) {  // inclusive scan of the run sums
    const unsigned add = t >= off ? run[cur][t - off] : 0u;
    run[cur ^ 1][t] = run[cur][t] + add;
    cur ^= 1;
    __syncthreads();
  }
  unsigned base = run[cur][t] - sum;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    hist[t * PER + i] = base;
    base += v[i];
  }
}

__global__ __launch_bounds__(kRsThreads) void rs_scatter_kernel(const unsigned* kin, const int* vin, int n,
                                                              int shift, const unsigned* offs, unsigned* kout,
                                                              int* vout) {
  __shared__ unsigned base[kRsBins];           // the digits' running output offsets
  __shared__ unsigned cnt[kRsWaves][kRsBins];  // a tile's digit counts per wavefront, then their prefixes
  __shared__ unsigned tot[kRsBins];            // a tile's digit counts
  const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
  for (int e = tid; e < kRsBins; e += kRsThreads) base[e] = offs[e * kRsBlocks + blockIdx.x];
  const int ch = rs_chunk(n), lo = min(n, (int)blockIdx.x * ch), hi = min(n, lo + ch);
  const unsigned long long below = (1ull << lane) - 1ull;  // the lanes before this one
  for (int t0 = lo; t0 < hi; t0 += kRsThreads) {
    for (int e = tid; e < kRsWaves * kRsBins; e += kRsThreads) cnt[e / kRsBins][e % kRsBins] = 0u;
    __syncthreads();
    const int i = t0 + tid;
    const bool valid = i < hi;  // the invalid lanes are the tile's last ones
    const unsigned key = valid ? kin[i] : 0u;
    const int val = valid ? (vin ? vin[i] : i) : 0;
    const unsigned d = rs_digit(key, shift);
    // the lanes of this wavefront holding the same digit
    unsigned long long same = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; b++) {
      const unsigned long long ones = __ballot((d >> b) & 1u);
      same &= ((d >> b) & 1u) ? ones : ~ones;
    }
    const unsigned rank = (unsigned)__popcll(same & below), group = (unsigned)__popcll(same);
    if (valid && rank == group - 1u) cnt[wave][d] = group;  // the group's last lane
    __syncthreads();
    for (int e = tid; e < kRsBins; e += kRsThreads) {  // prefixes over the wavefronts in order
      unsigned r = 0u;
#pragma unroll
      for (int w = 0; w < kRsWaves; w++) {
        const unsigned c = cnt[w][e];
        cnt[w][e] = r;
        r += c;
      }
      tot[e] = r;
    }
    __syncthreads();
    if (valid) {
      const unsigned pos = base[d] + cnt[wave][d] + rank;
      kout[pos] = key;
      vout[pos] = val;
    }
    __syncthreads();  // every read of base and cnt for this tile is done
    for (int e = tid; e < kRsBins; e += kRsThreads) base[e] += tot[e];
  }
}

}  // namespace

size_t sample_sort_temp_bytes(int V) {
  // a key and a value buffer for the passes between the input and the
  // output, and the digit counts
  return (size_t)V * (sizeof(unsigned) + sizeof(int)) + (size_t)kRsBins * kRsBlocks * sizeof(unsigned) + 256;
}

void sort_pairs_desc(const unsigned* keys, const int* vals, int n, unsigned* keys_out, int* vals_out, void* temp,
                     hipStream_t s) {
  if (n < 0 || n > kSortMax) ST_DIE("sort_pairs_desc: n out of range");
  if (n == 0) return;
  unsigned* tk = (unsigned*)temp;
  int* tv = (int*)(tk + n);
  unsigned* hist = (unsigned*)(((uintptr_t)(tv + n) + 255) & ~(uintptr_t)255);
  // passes 0..3: input -> temp -> output -> temp -> output
  const unsigned* kin = keys;
  const int* vin = vals;
  for (int pass = 0; pass < 4; pass++) {
    unsigned* ko = pass % 2 ? keys_out : tk;
    int* vo = pass % 2 ? vals_out : tv;
    const int shift = 8 * pass;
    hipLaunchKernelGGL(rs_hist_kernel, dim3(kRsBlocks), dim3(kRsThreads), 0, s, kin, n, shift, hist);
    hipLaunchKernelGGL(rs_scan_kernel, dim3(1), dim3(kRsScan), 0, s, hist);
    hipLaunchKernelGGL(rs_scatter_kernel, dim3(kRsBlocks), dim3(kRsThreads), 0, s, kin, vin, n, shift, hist, ko,
                       vo);
    kin = ko;
    vin = vo;
  }
  HIP_CHECK(hipGetLastError());
}

void sample(const SampleParams& p, hipStream_t s) {
  if (p.V <= 0) ST_DIE("sample needs a vocabulary");
  if (!(p.temperature >= 0.0f)) ST_DIE("sampling temperature must be >= 0");
  if (p.top_k < 0) ST_DIE("sampling top_k must be >= 0");
  const bool greedy = p.temperature == 0.0f;
  hipLaunchKernelGGL(sample_scale_kernel, dim3(kSB), dim3(kST), 0, s, p);
  if (greedy) {
    ArgmaxParams a{};
    a.x = p.y;
    a.n = p.V;
    a.part_v = p.argmax_v;
    a.part_i = p.argmax_i;
    a.out = p.out;
    a.seq = p.seq;
    a.seq_len = p.seq_len;
    a.pos_inc = p.pos_inc;
    argmax(a, s);
    return;
  }
  const bool filter = p.top_k > 0 || (p.top_p > 0.0f && p.top_p <= 1.0f);
  SampleParams q = p;
  if (!filter) q.keys = nullptr;  // keep every token: no sort
  hipLaunchKernelGGL(sample_exp_kernel, dim3(kSB), dim3(kST), 0, s, q);
  hipLaunchKernelGGL(sample_norm_kernel, dim3(kSB), dim3(kST), 0, s, q);
  if (filter) {
    if (p.sort_temp_bytes < sample_sort_temp_bytes(p.V)) ST_DIE("sample: sort scratch too small");
    sort_pairs_desc(p.keys, p.vals, p.V, p.keys_sorted, p.vals_sorted, p.sort_temp, s);
  }
  hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(kPick), 0, s, q);
  hipLaunchKernelGGL(sample_pick_kernel, dim3(1), dim3(kPick), 0, s, q);
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
