// act_order permutation (gptq_plus_utils.py:1046, 1050; classic GPTQ's argsort of diag(H),
// gptq_utils.py:73-76): perm = torch.argsort(key, descending=True), invperm = argsort(perm).
//
// torch's CPU argsort is not stable: with exactly equal keys (act_square of 4096 columns over
// 262144 tokens has dozens of exact ties) the order it returns is the one its sort algorithm
// produces, libstdc++'s std::sort (introsort) over (key, index) pairs with the comparator
// "a before b iff (a is NaN and b is not) or a > b".  The kernel reproduces that algorithm's
// result bit for bit, so that the quantization order -- and with it every code -- is the
// reference's:
//   * introsort loop: while a range has more than 16 elements, unless its depth budget
//     (2 floor(log2 n) at the top) is spent, move the median of (first+1, middle, last-1) to
//     first, partition [first+1, last) around it with the unguarded Hoare scheme, and continue
//     with both parts (budget - 1 each); a range whose budget is spent is heap-sorted
//     (make_heap + sort_heap);
//   * final insertion sort: it never moves an element across a partition boundary, so it is a
//     stable sort of each range left with at most 16 elements.
//
// The Hoare partition is computed in parallel.  With L_k the k-th position (from the left)
// whose element is not before the pivot and R_k the k-th position (from the right) whose
// element is not after it, the sequential scan swaps L_k with R_k for k = 1..K, K the largest
// k with L_k < R_k (a prefix, since L rises and R falls), and stops at
// min(L_{K+1}, R_K) (R_0 = infinity), which is the split point.  Pass 1 lists R_k, pass 2
// finds K and L_{K+1}, pass 3 swaps; every flag is read from elements no swap has touched.
//
// One workgroup of 16 waves.  Ranges above 512 elements are partitioned by the whole
// workgroup; smaller ones go to a list from which each wave takes ranges and finishes them
// alone (wave-wide partitions, leaf sorts, heap sort on one lane).  Keys and indices live in
// LDS up to 16384 columns, in the output buffers (global memory) above.
#include "rq_common.h"

#include <climits>

namespace {

constexpr int AS_THREADS = 1024;
constexpr int AS_WAVES = AS_THREADS / 64;
constexpr int AS_TB = 512;          // largest range a single wave takes
constexpr int AS_LEAF = 16;         // std::sort's insertion-sort threshold
constexpr int AS_SCAP = 512;        // small-range list capacity (drained when nearly full)
constexpr int AS_BCAP = 160;        // big-range stack (disjoint ranges of > 512: <= 128 at C <= 65536)
constexpr int AS_WSTACK = 40;       // per-wave stack (depth budget <= 32)
constexpr int AS_LDS_MAXC = 16384;
constexpr int AS_MAXC = 65536;

__device__ __forceinline__ bool before(float a, float b) { return (a != a && b == b) || (a > b); }

struct Range {
  int f, l, d;
};

template <typename IT>
struct Mem {
  float* key;
  IT* id;
  IT* rs;   // R_k positions of the current partition (per wave in the wave phase)
};

template <typename IT>
__device__ __forceinline__ void swap_elems(const Mem<IT>& M, int p, int q) {
  const float kp = M.key[p], kq = M.key[q];
  const IT ip = M.id[p], iq = M.id[q];
  M.key[p] = kq;
  M.key[q] = kp;
  M.id[p] = iq;
  M.id[q] = ip;
}

template <typename IT>
__device__ __forceinline__ bool before_at(const Mem<IT>& M, int p, int q) { return before(M.key[p], M.key[q]); }

// std::__move_median_to_first(result = f, a = f + 1, b = mid, c = l - 1)
template <typename IT>
__device__ void median_to_first(const Mem<IT>& M, int f, int l) {
  const int a = f + 1, b = f + (l - f) / 2, c = l - 1;
  if (before_at(M, a, b)) {
    if (before_at(M, b, c)) swap_elems(M, f, b);
    else if (before_at(M, a, c)) swap_elems(M, f, c);
    else swap_elems(M, f, a);
  } else if (before_at(M, a, c)) {
    swap_elems(M, f, a);
  } else if (before_at(M, b, c)) {
    swap_elems(M, f, c);
  } else {
    swap_elems(M, f, b);
  }
}

// libstdc++ heap primitives on [f, f + len) with the "before" comparator: std::__push_heap,
// std::__adjust_heap, make_heap, sort_heap (= std::partial_sort(first, last, last)).
template <typename IT>
__device__ void heap_push(const Mem<IT>& M, int f, int hole, int top, float vk, IT vi) {
  int parent = (hole - 1) / 2;
  while (hole > top && before(M.key[f + parent], vk)) {
    M.key[f + hole] = M.key[f + parent];
    M.id[f + hole] = M.id[f + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  M.key[f + hole] = vk;
  M.id[f + hole] = vi;
}

template <typename IT>
__device__ void heap_adjust(const Mem<IT>& M, int f, int hole, int len, float vk, IT vi) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (before(M.key[f + second], M.key[f + second - 1])) --second;
    M.key[f + hole] = M.key[f + second];
    M.id[f + hole] = M.id[f + second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    M.key[f + hole] = M.key[f + second - 1];
    M.id[f + hole] = M.id[f + second - 1];
    hole = second - 1;
  }
  heap_push(M, f, hole, top, vk, vi);
}

template <typename IT>
__device__ void heap_sort(const Mem<IT>& M, int f, int l) {
  const int len = l - f;
  if (len >= 2) {
    for (int parent = (len - 2) / 2;; --parent) {
      heap_adjust(M, f, parent, len, M.key[f + parent], M.id[f + parent]);
      if (parent == 0) break;
    }
  }
  for (int last = l; last - f > 1;) {
    --last;
    const float vk = M.key[last];
    const IT vi = M.id[last];
    M.key[last] = M.key[f];
    M.id[last] = M.id[f];
    heap_adjust(M, f, 0, last - f, vk, vi);
  }
}

__device__ __forceinline__ void wave_sync_mem() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int prefix_count(unsigned long long mask) {
  return __popcll(mask & ((1ull << lane_id()) - 1ull));
}

// ---- one wave ------------------------------------------------------------------------------

// Stable sort of a leaf of at most 16 elements (the final insertion sort's effect on it).
template <typename IT>
__device__ void wave_leaf_sort(const Mem<IT>& M, int f, int n) {
  const int lane = lane_id();
  const bool on = lane < n;
  const float k = on ? M.key[f + lane] : 0.0f;
  const IT id = on ? M.id[f + lane] : IT(0);
  int pos = 0;
  for (int j = 0; j < n; ++j) {
    const float kj = __shfl(k, j);
    pos += before(kj, k) ? 1 : 0;
    pos += (j < lane && !before(kj, k) && !before(k, kj)) ? 1 : 0;
  }
  wave_sync_mem();
  if (on) {
    M.key[f + pos] = k;
    M.id[f + pos] = id;
  }
  wave_sync_mem();
}

// Unguarded Hoare partition of [f + 1, l) around the pivot at f; returns the split point.
template <typename IT>
__device__ int wave_partition(const Mem<IT>& M, IT* rs, int f, int l) {
  const int lane = lane_id();
  const float pk = M.key[f];
  // pass 1: R_k from the right
  int nrs = 0;
  for (int base = l - 1; base >= f + 1; base -= 64) {
    const int p = base - lane;
    const bool fl = p >= f + 1 && !before(pk, M.key[p]);
    const unsigned long long m = __ballot(fl);
    if (fl) rs[nrs + prefix_count(m)] = (IT)p;
    nrs += __popcll(m);
  }
  wave_sync_mem();
  // pass 2: K and L_{K+1}
  int nls = 0, K = -1, lnext = INT_MAX;
  for (int base = f + 1; base < l && K < 0; base += 64) {
    const int p = base + lane;
    const bool fl = p < l && !before(M.key[p], pk);
    const unsigned long long m = __ballot(fl);
    const int k = nls + prefix_count(m);
    const bool swp = fl && k < nrs && p < (int)rs[max(0, min(k, nrs - 1))];
    const unsigned long long fail = __ballot(fl && !swp);
    if (fail) {
      const int first = __ffsll((long long)fail) - 1;   // lowest lane: smallest position and rank
      K = __shfl(k, first);
      lnext = __shfl(p, first);
    }
    nls += __popcll(m);
  }
  if (K < 0) K = nls;
  // pass 3: swap L_k and R_k for k < K (0-based ranks); positions <= L_K are untouched by the
  // swaps' right-hand writes, which all lie at or beyond R_K > L_K
  nls = 0;
  for (int base = f + 1; base < l && nls < K; base += 64) {
    const int p = base + lane;
    const bool fl = p < l && !before(M.key[p], pk);
    const unsigned long long m = __ballot(fl);
    const int k = nls + prefix_count(m);
    wave_sync_mem();
    if (fl && k < K) swap_elems(M, p, (int)rs[k]);
    wave_sync_mem();
    nls += __popcll(m);
  }
  int cut = (K >= 1) ? (int)rs[K - 1] : INT_MAX;
  if (lnext < cut) cut = lnext;
  // the two parts are non-empty for any consistent input; clamp so that the loop always ends
  return max(f + 1, min(cut, l - 1));
}

template <typename IT>
__device__ void wave_introsort(const Mem<IT>& M, IT* rs, Range* stack, Range r) {
  const int lane = lane_id();
  int sp = 0;
  for (;;) {
    int f = r.f, l = r.l, d = r.d;
    bool heaped = false;
    while (l - f > AS_LEAF) {
      if (d == 0) {
        if (lane == 0) heap_sort(M, f, l);
        wave_sync_mem();
        heaped = true;
        break;
      }
      --d;
      if (lane == 0) median_to_first(M, f, l);
      wave_sync_mem();
      const int cut = wave_partition(M, rs, f, l);
      if (sp < AS_WSTACK) {
        if (lane == 0) stack[sp] = Range{cut, l, d};
        ++sp;
      }
      wave_sync_mem();
      l = cut;
    }
    if (!heaped && l - f > 1) wave_leaf_sort(M, f, l - f);
    if (sp == 0) break;
    --sp;
    r = stack[sp];
  }
}

// ---- whole workgroup -----------------------------------------------------------------------

struct Shared {
  Range big[AS_BCAP];
  Range small[AS_SCAP];
  Range wstack[AS_WAVES][AS_WSTACK];
  int nbig, nsmall, head;
  int cnt[AS_WAVES];
  int nrs, nls, K, lnext, cut;
};

// Exclusive offset of this thread's flag among the workgroup's flags, and the total.
__device__ __forceinline__ int block_offset(Shared& S, bool fl, int* total) {
  const int wave = threadIdx.x >> 6;
  const unsigned long long m = __ballot(fl);
  if (lane_id() == 0) S.cnt[wave] = __popcll(m);
  __syncthreads();
  int off = 0, tot = 0;
  for (int w = 0; w < AS_WAVES; ++w) {
    const int c = S.cnt[w];
    off += (w < wave) ? c : 0;
    tot += c;
  }
  *total = tot;
  return off + prefix_count(m);
}

template <typename IT>
__device__ int block_partition(const Mem<IT>& M, Shared& S, int f, int l) {
  const int tid = threadIdx.x;
  const float pk = M.key[f];
  int nrs = 0;
  for (int base = l - 1; base >= f + 1; base -= AS_THREADS) {
    const int p = base - tid;
    const bool fl = p >= f + 1 && !before(pk, M.key[p]);
    int tot;
    const int off = block_offset(S, fl, &tot);
    if (fl) M.rs[nrs + off] = (IT)p;
    nrs += tot;
    __syncthreads();
  }
  if (tid == 0) {
    S.K = -1;
    S.lnext = INT_MAX;
  }
  __syncthreads();
  int nls = 0;
  for (int base = f + 1; base < l; base += AS_THREADS) {
    const int p = base + tid;
    const bool fl = p < l && !before(M.key[p], pk);
    int tot;
    const int k = nls + block_offset(S, fl, &tot);
    const bool swp = fl && k < nrs && p < (int)M.rs[max(0, min(k, nrs - 1))];
    if (fl && !swp) atomicMin(&S.lnext, p);
    __syncthreads();
    if (fl && !swp && p == S.lnext) S.K = k;
    nls += tot;
    __syncthreads();
    if (S.K >= 0) break;
  }
  const int K = (S.K >= 0) ? S.K : nls;
  nls = 0;
  for (int base = f + 1; base < l && nls < K; base += AS_THREADS) {
    const int p = base + tid;
    const bool fl = p < l && !before(M.key[p], pk);
    int tot;
    const int k = nls + block_offset(S, fl, &tot);
    __syncthreads();
    if (fl && k < K) swap_elems(M, p, (int)M.rs[k]);
    __syncthreads();
    nls += tot;
  }
  int cut = (K >= 1) ? (int)M.rs[K - 1] : INT_MAX;
  if (S.lnext < cut) cut = S.lnext;
  __syncthreads();
  return max(f + 1, min(cut, l - 1));
}

template <typename IT>
__device__ void push_range(Shared& S, Range r) {
  if (r.l - r.f > AS_TB && r.d > 0) {
    S.big[S.nbig++] = r;
  } else {
    S.small[S.nsmall++] = r;
  }
}

template <typename IT>
__device__ void argsort_body(const float* __restrict__ keys_in, int C, const Mem<IT>& M, Shared& S) {
  const int tid = threadIdx.x;
  for (int i = tid; i < C; i += AS_THREADS) {
    M.key[i] = keys_in[i];
    M.id[i] = (IT)i;
  }
  if (tid == 0) {
    int lg = 0;
    while ((2 << lg) <= C) ++lg;   // floor(log2 C)
    S.nbig = 0;
    S.nsmall = 0;
    if (C > 1) push_range<IT>(S, Range{0, C, 2 * lg});
  }
  __syncthreads();
  for (;;) {
    // whole-workgroup partitions of the big ranges, until none is left or the list fills
    while (S.nbig > 0 && S.nsmall <= AS_SCAP - 2) {
      const Range r = S.big[S.nbig - 1];
      __syncthreads();
      if (tid == 0) {
        --S.nbig;
        median_to_first(M, r.f, r.l);
      }
      __syncthreads();
      const int cut = block_partition(M, S, r.f, r.l);
      if (tid == 0) {
        push_range<IT>(S, Range{cut, r.l, r.d - 1});
        push_range<IT>(S, Range{r.f, cut, r.d - 1});
      }
      __syncthreads();
    }
    // every wave finishes small ranges from the list
    if (tid == 0) S.head = 0;
    __syncthreads();
    const int wave = tid >> 6;
    IT* rs = M.rs + wave * AS_TB;
    for (;;) {
      int idx = 0;
      if (lane_id() == 0) idx = atomicAdd(&S.head, 1);
      idx = __shfl(idx, 0);
      if (idx >= S.nsmall) break;
      const Range r = S.small[idx];
      if (r.l - r.f > AS_TB) {          // a big range whose depth budget is spent
        if (lane_id() == 0) heap_sort(M, r.f, r.l);
        wave_sync_mem();
      } else {
        wave_introsort(M, rs, S.wstack[wave], r);
      }
    }
    __syncthreads();
    if (tid == 0) S.nsmall = 0;
    __syncthreads();
    if (S.nbig == 0) break;
  }
}

// Keys and indices in LDS (C <= 16384).
__global__ __launch_bounds__(AS_THREADS) void k_argsort_lds(const float* __restrict__ key, int C,
                                                            int64_t* __restrict__ perm,
                                                            int64_t* __restrict__ invperm) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  __shared__ Shared S;
  const int nrs = max(C, AS_WAVES * AS_TB);
  Mem<uint16_t> M;
  M.key = reinterpret_cast<float*>(dyn);
  M.id = reinterpret_cast<uint16_t*>(dyn + 4 * (size_t)C);
  M.rs = reinterpret_cast<uint16_t*>(dyn + 6 * (size_t)C);
  (void)nrs;
  argsort_body<uint16_t>(key, C, M, S);
  __syncthreads();
  for (int i = threadIdx.x; i < C; i += AS_THREADS) {
    const int src = M.id[i];
    perm[i] = src;
    invperm[src] = i;
  }
}

// Keys and indices in the output buffers (C <= 65536): perm holds the keys and indices, invperm
// the partition lists; the result is written out at the end through a copy of the indices.
__global__ __launch_bounds__(AS_THREADS) void k_argsort_global(const float* __restrict__ key, int C,
                                                               int64_t* __restrict__ perm,
                                                               int64_t* __restrict__ invperm) {
  __shared__ Shared S;
  Mem<int32_t> M;
  M.key = reinterpret_cast<float*>(perm);
  M.id = reinterpret_cast<int32_t*>(perm) + C;
  M.rs = reinterpret_cast<int32_t*>(invperm);
  argsort_body<int32_t>(key, C, M, S);
  __syncthreads();
  int32_t* idcopy = reinterpret_cast<int32_t*>(invperm);
  for (int i = threadIdx.x; i < C; i += AS_THREADS) idcopy[i] = M.id[i];
  __syncthreads();
  for (int i = threadIdx.x; i < C; i += AS_THREADS) perm[i] = idcopy[i];
  __syncthreads();
  for (int i = threadIdx.x; i < C; i += AS_THREADS) invperm[perm[i]] = i;
}

size_t lds_bytes(int C) { return 6 * (size_t)C + 2 * (size_t)(C > AS_WAVES * AS_TB ? C : AS_WAVES * AS_TB); }

}  // namespace

extern "C" int rq_act_order_perm(const float* act_sq, int C, int64_t* perm, int64_t* invperm, void* stream) {
  if (!act_sq || !perm || !invperm || C <= 0 || C > AS_MAXC) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (C <= AS_LDS_MAXC) {
    const size_t lds = lds_bytes(C);
    static bool attr_set[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return RQ_EHIP;
    if (dev < 0 || dev >= 64) return RQ_EINVAL;
    if (!attr_set[dev]) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_argsort_lds),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes(AS_LDS_MAXC)) != hipSuccess)
        return RQ_EHIP;
      attr_set[dev] = true;
    }
    hipLaunchKernelGGL(k_argsort_lds, dim3(1), dim3(AS_THREADS), lds, s, act_sq, C, perm, invperm);
  } else {
    hipLaunchKernelGGL(k_argsort_global, dim3(1), dim3(AS_THREADS), 0, s, act_sq, C, perm, invperm);
  }
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}
