// Order-exact top-k selection of torch's CPU topk.
//
// The bank decisions of the reference depend on the exact output order of
// torch.topk on CPU, ties included:
//   - candidate choice: topk(g_e, k, sorted=False) (memory_banks.py:486-491)
//     and the exact bank uses the first Te of that order (:503-510);
//   - LRU victims: topk(rank_key, k, largest=False, sorted=True) (:663).
// torch's CPU kernel (ATen/native/TopKImpl.h) fills (value, index) pairs
// and runs
//   k * 64 <= n : std::partial_sort(first, first + k, last, comp)
//   otherwise   : std::nth_element(first, first + k - 1, last, comp) and,
//                 when sorted, std::sort(first, first + k - 1, comp)
// with comp(x, y) = (isnan(x) && !isnan(y)) || x > y for largest (and the
// mirrored form for smallest), then reads the first k pairs.  The order of
// equal keys is whatever those libstdc++ algorithms leave, so the steps
// below follow them one for one: introselect (median-of-three pivot moved
// to the front, unguarded Hoare partition, depth limit 2*floor(log2 n),
// insertion sort below 4 elements, heap select past the depth limit),
// introsort (threshold 16, then a final insertion sort) and the binary-heap
// routines (sift-down to a leaf then sift-up, as in __adjust_heap).  The
// code is written over an index range of a plain array so it compiles for
// host and device alike.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coda {
namespace sel {

template <typename V>
struct Item {
  V v;
  int64_t i;
};

template <typename V>
__host__ __device__ inline bool is_nan(V x) {
  return x != x;
}

// comp(x, y): "x goes before y"
template <typename V>
struct Before {
  bool largest;
  __host__ __device__ inline bool operator()(const Item<V>& x, const Item<V>& y) const {
    if (largest) return (is_nan(x.v) && !is_nan(y.v)) || (x.v > y.v);
    return (!is_nan(x.v) && is_nan(y.v)) || (x.v < y.v);
  }
};

template <typename V>
__host__ __device__ inline void swap_items(Item<V>* a, int64_t x, int64_t y) {
  Item<V> t = a[x];
  a[x] = a[y];
  a[y] = t;
}

__host__ __device__ inline int floor_log2(int64_t n) {
  int k = 0;
  while (n > 1) {
    n >>= 1;
    ++k;
  }
  return k;
}

// ---------------------------------------------------------------- heaps
// Heap over a[first, first + len) ordered by `before` (max-heap w.r.t. it).
template <typename V, typename C>
__host__ __device__ inline void heap_sift_up(Item<V>* a, int64_t first, int64_t hole, int64_t top,
                                             Item<V> value, const C& before) {
  int64_t parent = (hole - 1) / 2;
  while (hole > top && before(a[first + parent], value)) {
    a[first + hole] = a[first + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a[first + hole] = value;
}

template <typename V, typename C>
__host__ __device__ inline void heap_adjust(Item<V>* a, int64_t first, int64_t hole, int64_t len,
                                            Item<V> value, const C& before) {
  const int64_t top = hole;
  int64_t child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (before(a[first + child], a[first + child - 1])) child--;
    a[first + hole] = a[first + child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    a[first + hole] = a[first + child - 1];
    hole = child - 1;
  }
  heap_sift_up(a, first, hole, top, value, before);
}

template <typename V, typename C>
__host__ __device__ inline void heap_make(Item<V>* a, int64_t first, int64_t last, const C& before) {
  const int64_t len = last - first;
  if (len < 2) return;
  int64_t parent = (len - 2) / 2;
  while (true) {
    Item<V> value = a[first + parent];
    heap_adjust(a, first, parent, len, value, before);
    if (parent == 0) return;
    parent--;
  }
}

// Move the heap top to `result` and re-heap [first, last) with the old
// value of `result`.
template <typename V, typename C>
__host__ __device__ inline void heap_pop_to(Item<V>* a, int64_t first, int64_t last, int64_t result,
                                            const C& before) {
  Item<V> value = a[result];
  a[result] = a[first];
  heap_adjust(a, first, (int64_t)0, last - first, value, before);
}

template <typename V, typename C>
__host__ __device__ inline void heap_select(Item<V>* a, int64_t first, int64_t middle, int64_t last,
                                            const C& before) {
  heap_make(a, first, middle, before);
  for (int64_t i = middle; i < last; ++i)
    if (before(a[i], a[first])) heap_pop_to(a, first, middle, i, before);
}

template <typename V, typename C>
__host__ __device__ inline void heap_sort(Item<V>* a, int64_t first, int64_t last, const C& before) {
  while (last - first > 1) {
    --last;
    heap_pop_to(a, first, last, last, before);
  }
}

// ---------------------------------------------------------------- pieces
template <typename V, typename C>
__host__ __device__ inline void median_to_first(Item<V>* a, int64_t result, int64_t x, int64_t y,
                                                int64_t z, const C& before) {
  if (before(a[x], a[y])) {
    if (before(a[y], a[z])) swap_items(a, result, y);
    else if (before(a[x], a[z])) swap_items(a, result, z);
    else swap_items(a, result, x);
  } else if (before(a[x], a[z])) {
    swap_items(a, result, x);
  } else if (before(a[y], a[z])) {
    swap_items(a, result, z);
  } else {
    swap_items(a, result, y);
  }
}

template <typename V, typename C>
__host__ __device__ inline int64_t partition_unguarded(Item<V>* a, int64_t first, int64_t last,
                                                       int64_t pivot, const C& before) {
  while (true) {
    while (before(a[first], a[pivot])) ++first;
    --last;
    while (before(a[pivot], a[last])) --last;
    if (!(first < last)) return first;
    swap_items(a, first, last);
    ++first;
  }
}

template <typename V, typename C>
__host__ __device__ inline int64_t partition_pivot(Item<V>* a, int64_t first, int64_t last,
                                                   const C& before) {
  const int64_t mid = first + (last - first) / 2;
  median_to_first(a, first, first + 1, mid, last - 1, before);
  return partition_unguarded(a, first + 1, last, first, before);
}

template <typename V, typename C>
__host__ __device__ inline void linear_insert_unguarded(Item<V>* a, int64_t last, const C& before) {
  Item<V> value = a[last];
  int64_t next = last - 1;
  while (before(value, a[next])) {
    a[last] = a[next];
    last = next;
    --next;
  }
  a[last] = value;
}

template <typename V, typename C>
__host__ __device__ inline void insertion_sort(Item<V>* a, int64_t first, int64_t last, const C& before) {
  if (first == last) return;
  for (int64_t i = first + 1; i != last; ++i) {
    if (before(a[i], a[first])) {
      Item<V> value = a[i];
      for (int64_t j = i; j > first; --j) a[j] = a[j - 1];
      a[first] = value;
    } else {
      linear_insert_unguarded(a, i, before);
    }
  }
}

// ---------------------------------------------------------------- algorithms
template <typename V, typename C>
__host__ __device__ inline void nth_element(Item<V>* a, int64_t first, int64_t nth, int64_t last,
                                            const C& before) {
  if (first == last || nth == last) return;
  int depth = floor_log2(last - first) * 2;
  while (last - first > 3) {
    if (depth == 0) {
      heap_select(a, first, nth + 1, last, before);
      swap_items(a, first, nth);
      return;
    }
    --depth;
    const int64_t cut = partition_pivot(a, first, last, before);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  insertion_sort(a, first, last, before);
}

template <typename V, typename C>
__host__ __device__ inline void partial_sort(Item<V>* a, int64_t first, int64_t middle, int64_t last,
                                             const C& before) {
  heap_select(a, first, middle, last, before);
  heap_sort(a, first, middle, before);
}

// Introsort without recursion on the right part replaced: the left part
// loops, the right part recurses exactly like __introsort_loop.  The
// recursion depth is bounded by 2*floor(log2 n); an explicit stack keeps it
// device friendly.
template <typename V, typename C>
__host__ __device__ inline void sort(Item<V>* a, int64_t first, int64_t last, const C& before) {
  if (first == last) return;
  // each partition level pushes two frames and pops one, and levels are
  // bounded by the depth limit 2*floor(log2 n) <= 40 for n <= 2^20
  struct Frame {
    int32_t first, last, depth;
  };
  Frame stack[48];
  int sp = 0;
  stack[sp++] = Frame{(int32_t)first, (int32_t)last, floor_log2(last - first) * 2};
  while (sp > 0) {
    Frame f = stack[--sp];
    // __introsort_loop(f.first, f.last, f.depth): iterate on [first, cut),
    // recurse into [cut, last) before continuing
    int64_t lo = f.first, hi = f.last;
    int depth = f.depth;
    // The recursive call on [cut, hi) happens before the loop continues on
    // [lo, cut); both touch disjoint ranges, so deferring the left part
    // after the right part (LIFO) preserves the sequence of operations on
    // each range.  Push the left continuation first, then the right call.
    if (hi - lo > 16) {
      if (depth == 0) {
        partial_sort(a, lo, hi, hi, before);
        continue;
      }
      --depth;
      const int64_t cut = partition_pivot(a, lo, hi, before);
      stack[sp++] = Frame{(int32_t)lo, (int32_t)cut, depth};  // loop continuation, runs after the right part
      stack[sp++] = Frame{(int32_t)cut, (int32_t)hi, depth};  // recursive call, runs first
    }
  }
  // __final_insertion_sort
  if (last - first > 16) {
    insertion_sort(a, first, first + 16, before);
    for (int64_t i = first + 16; i != last; ++i) linear_insert_unguarded(a, i, before);
  } else {
    insertion_sort(a, first, last, before);
  }
}

// torch CPU topk order over a[0, n): afterwards a[0, k) holds the result.
template <typename V>
__host__ __device__ inline void topk_order(Item<V>* a, int64_t n, int64_t k, bool largest, bool sorted) {
  if (k == 0) return;
  Before<V> before{largest};
  if (k * 64 <= n) {
    partial_sort(a, (int64_t)0, k, n, before);
  } else {
    nth_element(a, (int64_t)0, k - 1, n, before);
    if (sorted) sort(a, (int64_t)0, k - 1, before);
  }
}

}  // namespace sel
}  // namespace coda
