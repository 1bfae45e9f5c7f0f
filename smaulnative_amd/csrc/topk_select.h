// Top-k selection order of the reference router (model.py:564, torch.topk on
// the CPU, sorted=True, largest=True).
//
// torch's CPU top-k (ATen/native/TopKImpl.h, torch 2.x) builds (value, index)
// pairs and, whenever k * 64 > n (true for every router width below 64),
// calls std::nth_element(q, q + k - 1, q + n, cmp) followed by
// std::sort(q, q + k - 1, cmp) (otherwise std::partial_sort(q, q + k, q + n,
// cmp)), where cmp(a, b) = (isnan(a) && !isnan(b)) ||
// a > b compares values only.  Between equal values the result therefore
// depends on the exact steps of the C++ library's introselect / introsort, not
// on the indices: e.g. four equal probabilities with k = 2 select {2, 3}.
//
// The steps below restate GNU libstdc++'s published algorithm (stl_algo.h /
// stl_heap.h, unchanged in this respect from GCC 4.x through GCC 14, which
// builds the torch wheels): introselect with a median-of-three pivot moved to
// the front and an unguarded Hoare partition, a heap-select fallback at depth
// 2*floor(log2 n), and a final insertion sort for ranges of at most 3; sort is
// introsort with threshold 16 and a final insertion sort.  Written as plain
// functions over an array so one copy serves the GPU router and the host
// self-test (smaul_selftest_topk).
#pragma once
#include <stdint.h>

#ifdef __HIPCC__
#define SMAUL_HD __host__ __device__
#else
#define SMAUL_HD
#endif

namespace smaul_topk {

struct Pair {
  float v;
  int i;
};

SMAUL_HD inline bool isnan_(float x) { return x != x; }
// cmp(a, b): a goes before b.
SMAUL_HD inline bool cmp(const Pair& a, const Pair& b) {
  return (isnan_(a.v) && !isnan_(b.v)) || (a.v > b.v);
}
SMAUL_HD inline void swp(Pair* a, Pair* b) {
  Pair t = *a;
  *a = *b;
  *b = t;
}
SMAUL_HD inline int lg(int n) {  // floor(log2(n)), n >= 1
  int r = 0;
  while (n > 1) {
    n >>= 1;
    ++r;
  }
  return r;
}

SMAUL_HD inline void push_heap(Pair* first, int hole, int top, Pair value) {
  int parent = (hole - 1) / 2;
  while (hole > top && cmp(first[parent], value)) {
    first[hole] = first[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  first[hole] = value;
}

SMAUL_HD inline void adjust_heap(Pair* first, int hole, int len, Pair value) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (cmp(first[second], first[second - 1])) second--;
    first[hole] = first[second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    first[hole] = first[second - 1];
    hole = second - 1;
  }
  push_heap(first, hole, top, value);
}

SMAUL_HD inline void make_heap(Pair* first, int len) {
  if (len < 2) return;
  int parent = (len - 2) / 2;
  while (true) {
    Pair value = first[parent];
    adjust_heap(first, parent, len, value);
    if (parent == 0) return;
    parent--;
  }
}

// pop the heap top into *result, re-heapifying [first, first+len)
SMAUL_HD inline void pop_heap(Pair* first, int len, Pair* result) {
  Pair value = *result;
  *result = first[0];
  adjust_heap(first, 0, len, value);
}

SMAUL_HD inline void heap_select(Pair* first, int middle, int last) {
  make_heap(first, middle);
  for (int i = middle; i < last; ++i)
    if (cmp(first[i], first[0])) pop_heap(first, middle, first + i);
}

SMAUL_HD inline void sort_heap(Pair* first, int len) {
  while (len > 1) {
    --len;
    pop_heap(first, len, first + len);
  }
}

SMAUL_HD inline void move_median_to_first(Pair* result, Pair* a, Pair* b, Pair* c) {
  if (cmp(*a, *b)) {
    if (cmp(*b, *c))
      swp(result, b);
    else if (cmp(*a, *c))
      swp(result, c);
    else
      swp(result, a);
  } else if (cmp(*a, *c)) {
    swp(result, a);
  } else if (cmp(*b, *c)) {
    swp(result, c);
  } else {
    swp(result, b);
  }
}

// [first, last) with pivot at *pivot, unguarded
SMAUL_HD inline int unguarded_partition(Pair* base, int first, int last, int pivot) {
  while (true) {
    while (cmp(base[first], base[pivot])) ++first;
    --last;
    while (cmp(base[pivot], base[last])) --last;
    if (!(first < last)) return first;
    swp(base + first, base + last);
    ++first;
  }
}

SMAUL_HD inline int unguarded_partition_pivot(Pair* base, int first, int last) {
  const int mid = first + (last - first) / 2;
  move_median_to_first(base + first, base + first + 1, base + mid, base + last - 1);
  return unguarded_partition(base, first + 1, last, first);
}

SMAUL_HD inline void unguarded_linear_insert(Pair* base, int last) {
  Pair val = base[last];
  int next = last - 1;
  while (cmp(val, base[next])) {
    base[last] = base[next];
    last = next;
    --next;
  }
  base[last] = val;
}

SMAUL_HD inline void insertion_sort(Pair* base, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i != last; ++i) {
    if (cmp(base[i], base[first])) {
      Pair val = base[i];
      for (int j = i; j > first; --j) base[j] = base[j - 1];
      base[first] = val;
    } else {
      unguarded_linear_insert(base, i);
    }
  }
}

SMAUL_HD inline void nth_element(Pair* base, int nth, int n) {
  if (n == 0 || nth == n) return;
  int first = 0, last = n;
  int depth = 2 * lg(n);
  while (last - first > 3) {
    if (depth == 0) {
      heap_select(base + first, nth + 1 - first, last - first);
      swp(base + first, base + nth);
      return;
    }
    --depth;
    const int cut = unguarded_partition_pivot(base, first, last);
    if (cut <= nth)
      first = cut;
    else
      last = cut;
  }
  insertion_sort(base, first, last);
}

// std::sort(base, base + n): introsort (threshold 16) + final insertion sort.
// The reference recursion on the right part is kept as an explicit stack.
SMAUL_HD inline void sort(Pair* base, int n) {
  if (n == 0) return;
  struct Frame {
    int first, last, depth;
  };
  Frame stack[16];
  int sp = 0;
  stack[sp++] = Frame{0, n, 2 * lg(n)};
  while (sp > 0) {
    Frame f = stack[--sp];
    int first = f.first, last = f.last, depth = f.depth;
    while (last - first > 16) {
      if (depth == 0) {
        heap_select(base + first, last - first, last - first);
        sort_heap(base + first, last - first);
        break;
      }
      --depth;
      const int cut = unguarded_partition_pivot(base, first, last);
      // introsort_loop(cut, last, depth) runs before the loop continues on
      // [first, cut); the two ranges are disjoint, so the order of doing them
      // does not change the result.
      if (sp < 16) stack[sp++] = Frame{cut, last, depth};
      last = cut;
    }
  }
  if (n > 16) {
    insertion_sort(base, 0, 16);
    for (int i = 16; i < n; ++i) unguarded_linear_insert(base, i);
  } else {
    insertion_sort(base, 0, n);
  }
}

// Selects the top-k of base[0..n) in torch's CPU order: afterwards base[0..k)
// holds the selected (value, index) pairs, sorted as torch returns them.
SMAUL_HD inline void topk(Pair* base, int n, int k) {
  if (k * 64 <= n) {  // std::partial_sort branch of TopKImpl.h
    heap_select(base, k, n);
    sort_heap(base, k);
    return;
  }
  nth_element(base, k - 1, n);
  sort(base, k - 1);
}

// topk for k <= 17: std::sort on at most 16 elements is a plain insertion
// sort (the introsort loop needs more than 16), so this is the same order as
// topk() without the explicit stack.
SMAUL_HD inline void topk_small(Pair* base, int n, int k) {
  if (k * 64 <= n) {
    heap_select(base, k, n);
    sort_heap(base, k);
    return;
  }
  nth_element(base, k - 1, n);
  insertion_sort(base, 0, k - 1);
}

}  // namespace smaul_topk
