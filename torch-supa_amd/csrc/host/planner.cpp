#include "planner.h"

#include <algorithm>
#include <numeric>
#include <stdexcept>

namespace supa {

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape) {
  std::vector<int64_t> st(shape.size());
  int64_t s = 1;
  for (size_t i = shape.size(); i-- > 0;) {
    st[i] = s;
    s *= std::max<int64_t>(shape[i], 1);
  }
  return st;
}

std::vector<int64_t> broadcast_shape(const std::vector<PlanOperand>& ops) {
  size_t nd = 0;
  bool any_input = false;
  for (const auto& o : ops)
    if (!o.is_output && !o.scalar) {
      nd = std::max(nd, o.sizes.size());
      any_input = true;
    }
  if (!any_input) {
    // no tensor inputs (fill): the first existing output gives the shape
    for (const auto& o : ops)
      if (o.is_output && !o.allocate) return o.sizes;
  }
  std::vector<int64_t> shape(nd, 1);
  for (const auto& o : ops) {
    if (o.is_output || o.scalar) continue;
    const size_t off = nd - o.sizes.size();
    for (size_t i = 0; i < o.sizes.size(); ++i) {
      const int64_t s = o.sizes[i];
      int64_t& t = shape[off + i];
      if (s == t || s == 1) continue;
      if (t == 1) {
        t = s;
        continue;
      }
      throw std::invalid_argument("The size of tensor a (" + std::to_string(t) + ") must match the size of tensor b (" +
                                  std::to_string(s) + ") at non-singleton dimension " + std::to_string(off + i));
    }
  }
  return shape;
}

Plan make_plan(const std::vector<PlanOperand>& ops) {
  Plan p;
  p.shape = broadcast_shape(ops);
  const int nd = (int)p.shape.size();
  const int nt = (int)ops.size();
  p.numel = 1;
  for (int64_t s : p.shape) p.numel *= s;

  // Per-operand strides, fastest-first ("reversed") and broadcast-aware.
  // rev_shape[i] is the size of tensor dim nd-1-i.
  std::vector<int64_t> rev_shape(nd);
  for (int i = 0; i < nd; ++i) rev_shape[i] = p.shape[nd - 1 - i];
  std::vector<std::vector<int64_t>> st(nt, std::vector<int64_t>(nd, 0));
  std::vector<bool> ignore(nt, false);  // operand does not vote on dim order
  for (int k = 0; k < nt; ++k) {
    const PlanOperand& o = ops[k];
    if (o.scalar || (o.is_output && o.allocate)) {
      ignore[k] = true;
      continue;
    }
    if (o.is_output && (int)o.sizes.size() != nd)
      throw std::invalid_argument("output rank does not match the broadcast shape");
    const int off = nd - (int)o.sizes.size();
    for (int i = 0; i < (int)o.sizes.size(); ++i) {
      const int rd = nd - 1 - (off + i);
      const int64_t sz = o.sizes[i];
      if (o.is_output && sz != p.shape[off + i]) throw std::invalid_argument("output shape does not match");
      st[k][rd] = (sz == 1 && p.shape[off + i] != 1) ? 0 : o.strides[i];
    }
  }

  // Dimension order: insertion sort over fastest-first dims with the
  // three-way comparison described in the header.
  std::vector<int> perm(nd);
  for (int i = 0; i < nd; ++i) perm[i] = i;  // perm[j] = original reversed dim at position j
  auto should_swap = [&](int d0, int d1) -> int {
    for (int k = 0; k < nt; ++k) {
      if (ignore[k]) continue;
      const int64_t s0 = st[k][d0], s1 = st[k][d1];
      if (s0 == 0 || s1 == 0) continue;
      if (s0 < s1) return -1;
      if (s0 > s1) return 1;
      if (rev_shape[d0] > rev_shape[d1]) return 1;
    }
    return 0;
  };
  for (int i = 1; i < nd; ++i) {
    int d1 = i;
    for (int d0 = i - 1; d0 >= 0; --d0) {
      const int c = should_swap(perm[d0], perm[d1]);
      if (c > 0) {
        std::swap(perm[d0], perm[d1]);
        d1 = d0;
      } else if (c < 0) {
        break;
      }
    }
  }

  // New outputs: dense in the permuted order.
  p.out_strides.assign(nt, {});
  for (int k = 0; k < nt; ++k) {
    if (!(ops[k].is_output && ops[k].allocate)) continue;
    std::vector<int64_t> tst(nd, 0);
    int64_t next = 1;
    for (int j = 0; j < nd; ++j) {
      const int rd = perm[j];
      tst[nd - 1 - rd] = next;
      next *= rev_shape[rd];
    }
    bool identity = true;
    for (int j = 0; j < nd; ++j) identity = identity && perm[j] == j;
    p.out_strides[k] = identity ? contiguous_strides(p.shape) : tst;
    for (int rd = 0; rd < nd; ++rd) st[k][rd] = p.out_strides[k][nd - 1 - rd];
  }

  // Iteration space in permuted order, then coalesce adjacent dims.
  std::vector<int64_t> sz(nd);
  std::vector<std::vector<int64_t>> pst(nt, std::vector<int64_t>(nd));
  for (int j = 0; j < nd; ++j) {
    sz[j] = rev_shape[perm[j]];
    for (int k = 0; k < nt; ++k) pst[k][j] = st[k][perm[j]];
  }
  std::vector<int64_t> csz;
  std::vector<std::vector<int64_t>> cst(nt);
  for (int j = 0; j < nd; ++j) {
    if (sz[j] == 1) continue;  // size-1 dims never move the index
    if (!csz.empty()) {
      bool merge = true;
      for (int k = 0; k < nt && merge; ++k) merge = pst[k][j] == cst[k].back() * csz.back();
      if (merge) {
        csz.back() *= sz[j];
        continue;
      }
    }
    csz.push_back(sz[j]);
    for (int k = 0; k < nt; ++k) cst[k].push_back(pst[k][j]);
  }
  if (p.numel == 0) {
    csz.assign(1, 0);
    for (int k = 0; k < nt; ++k) cst[k].assign(1, 0);
  }
  p.it_sizes = csz;
  p.it_strides = cst;
  return p;
}

}  // namespace supa
