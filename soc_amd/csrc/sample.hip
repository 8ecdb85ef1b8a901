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
// The kernels find S without a sequential scan. With q_i = row[i] / t, candidate i enters iff fewer than k earlier
// candidates j < i have q_j >= q_i, i.e. iff q_i is larger than T_i, the k-th largest of q_0..q_{i-1} (no threshold
// while fewer than k values precede). Two facts make this parallel:
//  - the multiset of the k largest values of any prefix is the top k of the per-chunk top-k lists of the chunks it
//    covers, and also the top k of the candidates of S it holds (the heap holds exactly these values);
//  - a value that is not above the k-th largest of a prefix cannot enter later, and cannot count against a later
//    candidate that is above it.
// k_topk_chunks writes each 2048-value chunk's top-k list. k_topk_accept (one block per chunk) merges the lists of
// the chunks before its own into the prefix top-k list L, then walks its chunk in rounds of 256 values: a value
// survives if it is above L[k-1]; a survivor enters iff L holds fewer than k values >= it minus the earlier
// survivors of its round that are >= it; L then absorbs the round's entrants. k_topk_gather concatenates the chunks'
// entrants. The host sorts the few candidates of S. For k = 1 the heap keeps the lowest index among the largest q,
// which k_topk_one finds in one launch.
#include "kernels.h"

namespace soc {
namespace {

constexpr int NT = 256;                // threads per block
constexpr int NW = NT / kWave;         // waves per block
constexpr int EPT = kSampleChunk / NT;  // values per thread in a chunk
constexpr int KM = kSampleMaxK;         // list length (k <= KM)

// Order of a value in the lists; NaN marks an empty list entry (it compares false with everything).
__device__ __forceinline__ float q_of(const float* row, int i, int V, float t) {
  return i < V ? __fdiv_rn(row[i], t) : __builtin_nanf("");
}

// Order-preserving block compaction: this thread's slot among the threads whose flag is set (in thread order), with
// the block's count in *total (the same in every thread). `ws` holds NW ints; two barriers.
__device__ __forceinline__ int block_compact(bool flag, int* ws, int* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint64_t b = __ballot(flag);
  if (lane == 0) ws[w] = __popcll(b);
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const int n = ws[u];
    off += u < w ? n : 0;
    tot += n;
  }
  __syncthreads();
  *total = tot;
  return off + __popcll(b & ((1ull << lane) - 1));
}

// Block: the top-k values (multiset, descending; entries past the chunk's size are NaN) of chunk c of q, and
// whether the chunk holds a NaN. Each wave extracts the k largest of its 512 values by repeated maxima; the four
// sorted wave lists are then merged by rank (a value's final position is its position in its own list plus the
// count of larger values in the other lists, ties going to the lower-numbered list).
__global__ __launch_bounds__(NT) void k_topk_chunks(const float* __restrict__ row, int V, float t, int k,
                                                     float* __restrict__ chunk_top, int* __restrict__ chunk_nan) {
  __shared__ float wl[NW][KM];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
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
  const int any_nan = __syncthreads_or(nan_seen);
  if (tid == 0) chunk_nan[c] = any_nan != 0;
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
    for (int u = 0; u < NW; ++u) {
      if (u == w) continue;
      for (int j = 0; j < k; ++j) {
        const float y = wl[u][j];
        pos += (u < w) ? (y >= x) : (y > x);
      }
    }
    if (pos < k) out[pos] = x;
  }
}

// Block c: writes the indices of the candidates of chunk c that enter the heap, in index order, to
// acc_idx[c * kSampleChunk ..] and their count to acc_cnt[c]. Dynamic LDS: c * k floats (the lists of chunks 0..c-1).
__global__ __launch_bounds__(NT) void k_topk_accept(const float* __restrict__ row, int V, float t, int k,
                                                     const float* __restrict__ chunk_top, int* __restrict__ acc_cnt,
                                                     int* __restrict__ acc_idx) {
  extern __shared__ float lists[];  // list j at lists[j * k], j < c
  __shared__ float q[kSampleChunk];
  __shared__ float rv[NT + 8];  // this round's survivors (values, in index order); 8 pad entries for the unrolled scan
  __shared__ int ri[NT];        // their positions in the chunk
  __shared__ float ev[NT];      // this round's entrants (values, in index order)
  __shared__ float lbuf[2][KM];
  __shared__ int ws[NW];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int c0 = c * kSampleChunk;
  const float qnan = __builtin_nanf("");
  for (int e = 0; e < EPT; ++e) q[e * NT + tid] = q_of(row, c0 + e * NT + tid, V, t);
  for (int j = tid; j < c * k; j += NT) lists[j] = chunk_top[static_cast<size_t>(j / k) * KM + j % k];
  if (tid < 8) rv[NT + tid] = qnan;
  __syncthreads();

  // prefix list: pairwise rank merges, list a = 2 span p absorbing list a + span; a group of g lanes (the power of
  // two >= k) merges one pair, entry gl of each list placed by lane gl
  int g = 1;
  while (g < k) g <<= 1;
  const int gpw = kWave / g, grp = lane / g, gl = lane % g;
  for (int span = 1; span < c; span <<= 1) {
    const int np = (c - span + 2 * span - 1) / (2 * span);  // pairs whose second list exists
    for (int base = 0; base < np; base += NW * gpw) {          // the same trip count in every thread
      const int p = base + w * gpw + grp;
      const bool act = p < np && gl < k;
      float* A = lists + static_cast<size_t>(2 * span * (act ? p : 0)) * k;
      const float* B = A + static_cast<size_t>(span) * k;
      float a = qnan, b = qnan;
      int pa = k, pb = k;
      if (act) {
        a = A[gl];
        b = B[gl];
        int ca = 0, cb = 0;
        for (int j = 0; j < k; ++j) {
          ca += B[j] > a;   // B's larger values go first
          cb += A[j] >= b;  // and A's equal ones too
        }
        if (a == a) pa = gl + ca;
        if (b == b) pb = gl + cb;
      }
      __syncthreads();
      if (act) A[gl] = qnan;
      __syncthreads();
      if (pa < k) A[pa] = a;
      if (pb < k) A[pb] = b;
      __syncthreads();
    }
  }

  float* L = lbuf[0];
  float* Ln = lbuf[1];
  if (tid < KM) L[tid] = (c > 0 && tid < k) ? lists[tid] : qnan;
  __syncthreads();
  int nacc = 0;
  for (int e = 0; e < EPT; ++e) {
    const float th = L[k - 1];
    const int li = e * NT + tid;
    const float x = q[li];
    const bool surv = x == x && !(x <= th);  // q is NaN past the row's end; no threshold while th is NaN
    int nr;
    const int r = block_compact(surv, ws, &nr);
    if (surv) {
      rv[r] = x;
      ri[r] = li;
    }
    __syncthreads();
    if (nr == 0) continue;
    // survivor tid: L's values >= it, then the earlier survivors' (values not above th are below it)
    bool enter = false;
    float v = qnan;
    int cl = 0;
    if (tid < nr) {
      v = rv[tid];
      for (int j = 0; j < k; ++j) cl += L[j] >= v;
      int cnt = cl;
      for (int j = 0; j < tid && cnt < k; j += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) cnt += (j + u < tid) & (rv[j + u] >= v);
      }
      enter = cnt < k;
    }
    int ne;
    const int m = block_compact(enter, ws, &ne);
    if (enter) {
      ev[m] = v;
      acc_idx[c0 + nacc + m] = c0 + ri[tid];
    }
    nacc += ne;
    __syncthreads();
    if (ne == 0) continue;
    // L <- top k of L and the entrants (order: value descending; L before entrants, entrants by index on ties)
    int pl = KM, pe = KM;
    float a = qnan;
    if (tid < k) {
      a = L[tid];
      if (a == a) {
        int cnt = tid;
        for (int j = 0; j < ne; ++j) cnt += ev[j] > a;
        pl = cnt;
      }
    }
    if (enter) {
      int cnt = cl;
      for (int j = 0; j < ne; ++j) {
        const float y = ev[j];
        cnt += (y > v) | ((y == v) & (j < m));
      }
      pe = cnt;
    }
    if (tid < KM) Ln[tid] = qnan;
    __syncthreads();
    if (pl < k) Ln[pl] = a;
    if (pe < k) Ln[pe] = v;
    __syncthreads();
    float* tmp = L;
    L = Ln;
    Ln = tmp;
  }
  if (tid == 0) acc_cnt[c] = nacc;
}

// Block c: copies chunk c's entrants after those of chunks 0..c-1: out[2 + 2 j] = index, out[3 + 2 j] = its raw
// logit's bits, for j < max_out. Block 0 writes out[0] = count of all entrants, out[1] = NaN seen.
__global__ __launch_bounds__(NT) void k_topk_gather(const float* __restrict__ row, int nch,
                                                     const int* __restrict__ chunk_nan,
                                                     const int* __restrict__ acc_cnt, const int* __restrict__ acc_idx,
                                                     int max_out, int* __restrict__ out) {
  __shared__ int red[2][NW];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  int before = 0, total = 0;
  bool nan_seen = false;
  for (int j = tid; j < nch; j += NT) {
    const int n = acc_cnt[j];
    before += j < c ? n : 0;
    total += n;
    nan_seen |= chunk_nan[j] != 0;
  }
  for (int o = 32; o > 0; o >>= 1) {
    before += __shfl_xor(before, o);
    total += __shfl_xor(total, o);
  }
  if (lane == 0) {
    red[0][w] = before;
    red[1][w] = total;
  }
  const int any_nan = __syncthreads_or(nan_seen);
  before = total = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    before += red[0][u];
    total += red[1][u];
  }
  const int n = acc_cnt[c];
  for (int r = tid; r < n; r += NT) {
    const int o = before + r;
    if (o < max_out) {
      const int i = acc_idx[static_cast<size_t>(c) * kSampleChunk + r];
      out[2 + 2 * o] = i;
      out[3 + 2 * o] = __float_as_int(row[i]);
    }
  }
  if (c == 0 && tid == 0) {
    out[0] = total;
    out[1] = any_nan != 0;
  }
}

// (value, index) order of the k = 1 search: a larger value, or an equal value at a lower index; index 0x7fffffff
// marks an empty candidate.
__device__ __forceinline__ bool first_max_better(float v, int i, float bv, int bi) {
  return i != 0x7fffffff && (bi == 0x7fffffff || v > bv || (v == bv && i < bi));
}

// Block-wide first maximum of (bv, bi); every thread gets it. sv / si hold NW entries.
__device__ __forceinline__ void block_first_max(float& bv, int& bi, float* sv, int* si) {
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (first_max_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[threadIdx.x / kWave] = bv;
    si[threadIdx.x / kWave] = bi;
  }
  __syncthreads();
  bv = sv[0];
  bi = si[0];
#pragma unroll
  for (int u = 1; u < NW; ++u)
    if (first_max_better(sv[u], si[u], bv, bi)) {
      bv = sv[u];
      bi = si[u];
    }
  __syncthreads();
}

// k = 1 in one launch. The one candidate partial_sort keeps is the lowest index among the largest q, so block c
// reduces chunk c to its (largest q, lowest index), publishes it, and the last block to arrive (counter zero before
// the launch, reset by that block) writes out[0] = 1, out[1] = NaN seen, out[2] = the index, out[3] = its raw logit's
// bits. Within a thread indices rise, so the strict `>` keeps the lowest index of equal values.
__global__ __launch_bounds__(NT) void k_topk_one(const float* __restrict__ row, int V, float t,
                                                  float* __restrict__ part_val, int* __restrict__ part_idx,
                                                  int* __restrict__ part_nan, int* __restrict__ counter,
                                                  int* __restrict__ out) {
  __shared__ float sv[NW];
  __shared__ int si[NW];
  __shared__ int last;
  const int c = blockIdx.x, nch = gridDim.x, tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  bool nan_seen = false;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = c * kSampleChunk + e * NT + tid;
    if (i < V) {
      const float x = __fdiv_rn(row[i], t);
      if (x != x) {
        nan_seen = true;
      } else if (bi == 0x7fffffff || x > bv) {
        bv = x;
        bi = i;
      }
    }
  }
  const int any_nan = __syncthreads_or(nan_seen);
  block_first_max(bv, bi, sv, si);
  if (tid == 0) {
    st_dev(part_val + c, bv);
    st_dev(part_idx + c, bi);
    st_dev(part_nan + c, any_nan != 0);
    wait_mem();  // the candidate is visible device-wide before it is counted
    last = atomicAdd(counter, 1) == nch - 1;
  }
  __syncthreads();
  if (!last) return;
  bv = -INFINITY;
  bi = 0x7fffffff;
  nan_seen = false;
  for (int b = tid; b < nch; b += NT) {
    const float pv = ld_dev(part_val + b);
    const int pi = ld_dev(part_idx + b);
    nan_seen |= ld_dev(part_nan + b) != 0;
    if (first_max_better(pv, pi, bv, bi)) {
      bv = pv;
      bi = pi;
    }
  }
  const int nan_all = __syncthreads_or(nan_seen);
  block_first_max(bv, bi, sv, si);
  if (tid == 0) {
    const int idx = bi == 0x7fffffff ? 0 : bi;  // no value at all: every entry NaN, reported by the flag
    out[0] = 1;
    out[1] = nan_all != 0;
    out[2] = idx;
    out[3] = __float_as_int(row[idx]);
    st_dev(counter, 0);
  }
}

}  // namespace

bool sample_device_fits(int V, int k) {
  if (V <= 0 || k <= 0 || k > KM) return false;
  const size_t nch = (static_cast<size_t>(V) + kSampleChunk - 1) / kSampleChunk;
  return nch * static_cast<size_t>(k) * 4 <= kSampleTreeBytes;
}

size_t sample_ws_bytes(int V) {
  const size_t nch = (static_cast<size_t>(V) + kSampleChunk - 1) / kSampleChunk;
  return 256 + nch * 4 * 2 + nch * KM * 4 + nch * kSampleChunk * 4;
}

hipError_t launch_sample_topk(const float* row, int V, float t, int k, void* ws, int* out, int max_out,
                              hipStream_t s) {
  if (!sample_device_fits(V, k) || max_out <= 0) return hipErrorInvalidValue;
  const int nch = (V + kSampleChunk - 1) / kSampleChunk;
  int* counter = static_cast<int*>(ws);
  int* chunk_nan = counter + 64;
  int* acc_cnt = chunk_nan + nch;
  float* chunk_top = reinterpret_cast<float*>(acc_cnt + nch);
  int* acc_idx = reinterpret_cast<int*>(chunk_top + static_cast<size_t>(nch) * KM);
  if (k == 1) {  // partials in the first entries of the lists' regions
    hipLaunchKernelGGL(k_topk_one, dim3(nch), dim3(NT), 0, s, row, V, t, chunk_top, acc_cnt, chunk_nan, counter, out);
    return hipGetLastError();
  }
  const size_t tree = static_cast<size_t>(nch) * k * 4;
  hipLaunchKernelGGL(k_topk_chunks, dim3(nch), dim3(NT), 0, s, row, V, t, k, chunk_top, chunk_nan);
  hipLaunchKernelGGL(k_topk_accept, dim3(nch), dim3(NT), tree, s, row, V, t, k, chunk_top, acc_cnt, acc_idx);
  hipLaunchKernelGGL(k_topk_gather, dim3(nch), dim3(NT), 0, s, row, nch, chunk_nan, acc_cnt, acc_idx, max_out, out);
  return hipGetLastError();
}

}  // namespace soc
