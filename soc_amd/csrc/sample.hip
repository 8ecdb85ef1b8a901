// sample.hip - top-k candidate selection on the device for the sampler (Mac/gpu/src/runtime/sampler.cpp:14-71).
//
// The reference copies the whole logits row to the host and runs
//   std::partial_sort(cand, cand + k, cand + V, [](l, r) { return row[l] / t > row[r] / t; })
// over cand = 0..V-1, then reports cand[0..k). That sort is a heap selection: the first k candidates form a heap,
// and candidate i >= k enters it (replacing the root) exactly when row[i] / t is larger than the current root, i.e.
// than the k-th largest value among candidates 0..i-1; every other candidate is never touched. Running the same
// std::partial_sort over only S = {0..k-1} followed by the candidates that enter, in index order, therefore repeats
// the same comparisons on the same heap and yields the same k candidates in the same order, ties included.
//
// The kernels find S without a sequential scan: with q_i = row[i] / t, candidate i >= k enters iff fewer than k
// earlier candidates j < i have q_j >= q_i. The row is cut into chunks of kChunk; for each chunk the top-k values
// of everything before it (a prefix list) bound which of its candidates can enter, and a survivor counts the
// prefix list plus its own chunk's earlier values. The host then sorts the few candidates of S.
#include "kernels.h"

namespace soc {
namespace {

constexpr int NT = 256;                // threads per block
constexpr int EPT = kSampleChunk / NT;  // elements per thread
constexpr int KM = kSampleMaxK;         // list length (k <= KM)

// Order of a value in the lists; NaN marks an empty list entry (it compares false with everything).
__device__ __forceinline__ float q_of(const float* row, int i, int V, float t) {
  return i < V ? __fdiv_rn(row[i], t) : __builtin_nanf("");
}

// Block: the top-k values (multiset, descending; entries past the chunk's size are NaN) of chunk c of q.
// Each wave extracts the k largest of its 512 values by repeated maxima; the four sorted wave lists are then
// merged by rank (a value's final position is its position in its own list plus the count of larger values in
// the other lists, ties going to the lower-numbered list).
__global__ __launch_bounds__(NT) void k_topk_chunks(const float* __restrict__ row, int V, float t, int k,
                                                     float* __restrict__ chunk_top, int* __restrict__ nan_flag) {
  __shared__ float wl[NT / kWave][KM];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float v[EPT];
  uint32_t present = 0;
  bool nan_seen = false;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    // wave w takes elements [512 w, 512 w + 512) of the chunk, lane-interleaved
    const int i = c * kSampleChunk + w * (kWave * EPT) + e * kWave + lane;
    v[e] = q_of(row, i, V, t);
    if (i < V) {
      if (v[e] != v[e]) nan_seen = true;
      else present |= 1u << e;
    }
  }
  if (nan_seen) atomicOr(nan_flag, 1);
  for (int r = 0; r < k; ++r) {
    float best = -INFINITY;
    int be = -1;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (((present >> e) & 1u) && (be < 0 || v[e] > best)) {
        best = v[e];
        be = e;
      }
    const uint64_t any = __ballot(be >= 0);
    if (any == 0) {
      if (lane == 0) wl[w][r] = __builtin_nanf("");
      continue;
    }
    // maximum over lanes that hold a value (-inf is a value here)
    float m = be >= 0 ? best : -INFINITY;
    m = wave_max(m);
    const uint64_t hit = __ballot(be >= 0 && best == m);
    const int src = __builtin_ctzll(hit);
    if (lane == src) present &= ~(1u << be);
    if (lane == 0) wl[w][r] = m;
  }
  for (int r = k; r < KM; ++r)
    if (lane == 0) wl[w][r] = __builtin_nanf("");
  __syncthreads();
  // merge: wave w places its own entry `lane`
  float* out = chunk_top + static_cast<size_t>(c) * KM;
  if (w == 0) out[lane] = __builtin_nanf("");  // KM == 64 entries, one per lane
  __syncthreads();
  const float x = wl[w][lane];
  if (lane < k && x == x) {
    int pos = lane;
    for (int u = 0; u < NT / kWave; ++u) {
      if (u == w) continue;
      for (int j = 0; j < k; ++j) {
        const float y = wl[u][j];
        pos += (u < w) ? (y >= x) : (y > x);
      }
    }
    if (pos < k) out[pos] = x;
  }
}

// One wave: prefix[c] = top-k values of chunks 0..c-1 (prefix[0] empty), by successive rank merges.
__global__ __launch_bounds__(kWave) void k_topk_prefix(const float* __restrict__ chunk_top, int nch, int k,
                                                        float* __restrict__ prefix) {
  __shared__ float cur[KM], nxt[KM];
  const int lane = threadIdx.x;
  cur[lane] = __builtin_nanf("");
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    prefix[static_cast<size_t>(c) * KM + lane] = cur[lane];
    if (c + 1 == nch) break;
    const float* b = chunk_top + static_cast<size_t>(c) * KM;
    const float a = cur[lane], bb = b[lane];
    nxt[lane] = __builtin_nanf("");
    __syncthreads();
    // the current list goes first on ties
    if (lane < k && a == a) {
      int pos = lane;
      for (int j = 0; j < k; ++j) pos += b[j] > a;
      if (pos < k) nxt[pos] = a;
    }
    if (lane < k && bb == bb) {
      int pos = lane;
      for (int j = 0; j < k; ++j) pos += cur[j] >= bb;
      if (pos < k) nxt[pos] = bb;
    }
    __syncthreads();
    cur[lane] = nxt[lane];
    __syncthreads();
  }
}

// Block c: flags the candidates of chunk c that enter the heap (i < k, or fewer than k earlier values >= q_i),
// and writes their indices, in index order, to acc_idx[c * kSampleChunk ..] with the count in acc_cnt[c].
__global__ __launch_bounds__(NT) void k_topk_accept(const float* __restrict__ row, int V, float t, int k,
                                                     const float* __restrict__ prefix, int* __restrict__ acc_cnt,
                                                     int* __restrict__ acc_idx) {
  __shared__ float q[kSampleChunk];
  __shared__ float pl[KM];
  __shared__ int wsum[NT / kWave];
  __shared__ int base;
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c0 = c * kSampleChunk;
  for (int e = 0; e < EPT; ++e) q[e * NT + tid] = q_of(row, c0 + e * NT + tid, V, t);
  if (tid < KM) pl[tid] = prefix[static_cast<size_t>(c) * KM + tid];
  if (tid == 0) base = 0;
  __syncthreads();
  const float theta = pl[k - 1];  // NaN while fewer than k values precede the chunk
  for (int e = 0; e < EPT; ++e) {
    const int li = e * NT + tid, i = c0 + li;
    const float x = q[li];
    bool enter = false;
    if (i < V && x == x) {
      if (i < k) {
        enter = true;
      } else if (theta != theta || x > theta) {
        int cnt = 0;
        for (int j = 0; j < k; ++j) cnt += pl[j] >= x;
        for (int j = 0; j < li && cnt < k; ++j) cnt += q[j] >= x;
        enter = cnt < k;
      }
    }
    // order-preserving compaction of this round (indices c0 + e * NT + tid ascend with tid)
    const uint64_t b = __ballot(enter);
    if (lane == 0) wsum[w] = __popcll(b);
    __syncthreads();
    int off = base;
    for (int u = 0; u < w; ++u) off += wsum[u];
    if (enter) acc_idx[c0 + off + __popcll(b & ((1ull << lane) - 1))] = i;
    __syncthreads();
    if (tid == 0) base += wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
  }
  if (tid == 0) acc_cnt[c] = base;
}

// One block: the per-chunk lists concatenated in chunk order, with their raw logits: out[0] = count, out[1] = NaN
// flag, out[2 ..] = indices (up to max_out), then max_out logits.
__global__ __launch_bounds__(NT) void k_topk_gather(const float* __restrict__ row, int nch,
                                                     const int* __restrict__ acc_cnt, const int* __restrict__ acc_idx,
                                                     const int* __restrict__ nan_flag, int max_out,
                                                     int* __restrict__ out) {
  __shared__ int off;
  if (threadIdx.x == 0) off = 0;
  __syncthreads();
  float* vals = reinterpret_cast<float*>(out + 2 + max_out);
  for (int c = 0; c < nch; ++c) {
    const int n = acc_cnt[c], o = off;
    for (int r = threadIdx.x; r < n; r += NT)
      if (o + r < max_out) {
        const int i = acc_idx[c * kSampleChunk + r];
        out[2 + o + r] = i;
        vals[o + r] = row[i];
      }
    __syncthreads();
    if (threadIdx.x == 0) off = o + n;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[0] = off;
    out[1] = *nan_flag;
  }
}

__global__ void k_zero_int(int* p) { *p = 0; }

}  // namespace

size_t sample_ws_bytes(int V) {
  const size_t nch = (static_cast<size_t>(V) + kSampleChunk - 1) / kSampleChunk;
  return 256 + nch * KM * 4 * 2 + nch * 4 + nch * kSampleChunk * 4;
}

hipError_t launch_sample_topk(const float* row, int V, float t, int k, void* ws, int* out, int max_out,
                              hipStream_t s) {
  if (V <= 0 || k <= 0 || k > KM || max_out <= 0) return hipErrorInvalidValue;
  const int nch = (V + kSampleChunk - 1) / kSampleChunk;
  char* p = static_cast<char*>(ws);
  int* nan_flag = reinterpret_cast<int*>(p);
  float* chunk_top = reinterpret_cast<float*>(p + 256);
  float* prefix = chunk_top + static_cast<size_t>(nch) * KM;
  int* acc_cnt = reinterpret_cast<int*>(prefix + static_cast<size_t>(nch) * KM);
  int* acc_idx = acc_cnt + nch;
  hipLaunchKernelGGL(k_zero_int, dim3(1), dim3(1), 0, s, nan_flag);
  hipLaunchKernelGGL(k_topk_chunks, dim3(nch), dim3(NT), 0, s, row, V, t, k, chunk_top, nan_flag);
  hipLaunchKernelGGL(k_topk_prefix, dim3(1), dim3(kWave), 0, s, chunk_top, nch, k, prefix);
  hipLaunchKernelGGL(k_topk_accept, dim3(nch), dim3(NT), 0, s, row, V, t, k, prefix, acc_cnt, acc_idx);
  hipLaunchKernelGGL(k_topk_gather, dim3(1), dim3(NT), 0, s, row, nch, acc_cnt, acc_idx, nan_flag, max_out, out);
  return hipGetLastError();
}

}  // namespace soc
