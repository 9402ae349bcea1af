// Fuzzes the iteration planner (csrc/host/planner.cpp, plain C++) for
// memory and undefined-behaviour errors under -fsanitize=address,undefined,
// and checks its plans by brute force: over random operand sets (ranks 0-6,
// broadcast, permuted, sliced, empty dims, immediate scalars, existing and
// new outputs), the coalesced iteration space must visit exactly the
// (output, input...) element tuples of the broadcast shape, each once, and a
// new output's strides must be dense in some dimension order.  Mismatched shapes must throw std::invalid_argument.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <random>
#include <stdexcept>
#include <vector>

#include "planner.h"

using supa::PlanOperand;
using Tuple = std::vector<int64_t>;

static void visit_logical(const std::vector<int64_t>& shape, const std::vector<std::vector<int64_t>>& strides,
                          std::vector<Tuple>& out) {
  const int nd = (int)shape.size();
  int64_t n = 1;
  for (int64_t s : shape) n *= s;
  std::vector<int64_t> idx(nd, 0);
  for (int64_t e = 0; e < n; ++e) {
    Tuple t;
    for (const auto& st : strides) {
      int64_t off = 0;
      for (int i = 0; i < nd; ++i) off += idx[i] * st[i];
      t.push_back(off);
    }
    out.push_back(t);
    for (int i = nd - 1; i >= 0; --i) {
      if (++idx[i] < shape[i]) break;
      idx[i] = 0;
    }
  }
}

static void visit_plan(const supa::Plan& p, int nt, std::vector<Tuple>& out) {
  const int nd = (int)p.it_sizes.size();
  int64_t n = 1;
  for (int64_t s : p.it_sizes) n *= s;
  std::vector<int64_t> idx(nd, 0);
  for (int64_t e = 0; e < n; ++e) {
    Tuple t;
    for (int k = 0; k < nt; ++k) {
      int64_t off = 0;
      for (int i = 0; i < nd; ++i) off += idx[i] * p.it_strides[k][i];
      t.push_back(off);
    }
    out.push_back(t);
    for (int i = 0; i < nd; ++i) {  // fastest first
      if (++idx[i] < p.it_sizes[i]) break;
      idx[i] = 0;
    }
  }
}

int main() {
  std::mt19937_64 rng(77);
  long plans = 0, throws = 0;
  for (int it = 0; it < 20000; ++it) {
    const int nd = (int)(rng() % 7);
    std::vector<int64_t> shape(nd);
    int64_t total = 1;
    for (auto& s : shape) {
      s = (rng() % 17 == 0) ? 0 : 1 + (int64_t)(rng() % 5);
      total *= s;
    }
    if (total > 5000) continue;
    const int nin = 1 + (int)(rng() % 3);
    std::vector<PlanOperand> ops(1 + nin);
    const bool new_out = rng() % 2;
    ops[0].is_output = true;
    ops[0].allocate = new_out;
    std::vector<std::vector<int64_t>> full(1 + nin, std::vector<int64_t>(nd, 0));  // strides on the broadcast shape
    auto dense_perm = [&](const std::vector<int64_t>& sz, std::vector<int64_t>& st) {
      std::vector<int> order(sz.size());
      for (size_t i = 0; i < sz.size(); ++i) order[i] = (int)i;
      std::shuffle(order.begin(), order.end(), rng);
      int64_t s = 1 + (int64_t)(rng() % 2);
      st.assign(sz.size(), 0);
      for (int i : order) {
        st[i] = s;
        s *= std::max<int64_t>(sz[i], 1) + (int64_t)(rng() % 2);
      }
    };
    for (int k = 1; k <= nin; ++k) {
      PlanOperand& o = ops[k];
      if (rng() % 9 == 0) {
        o.scalar = true;
        continue;
      }
      const int r = nd == 0 ? 0 : (int)(rng() % (nd + 1));  // trailing-aligned rank
      o.sizes.assign(shape.end() - r, shape.end());
      for (auto& s : o.sizes)
        if (s != 0 && rng() % 4 == 0) s = 1;  // broadcast dim
      if (r > 0 && rng() % 50 == 0 && o.sizes.back() > 1) o.sizes.back() += 1;  // a possible mismatch
      dense_perm(o.sizes, o.strides);
      for (int i = 0; i < r; ++i) {
        const int fd = nd - r + i;
        full[k][fd] = (o.sizes[i] == 1 && shape[fd] != 1) ? 0 : o.strides[i];
      }
    }
    bool all_scalar_inputs = true;
    for (int k = 1; k <= nin; ++k) all_scalar_inputs = all_scalar_inputs && ops[k].scalar;
    if (all_scalar_inputs && new_out) continue;  // no shape to take
    // the inputs' broadcast shape (numpy rules); an existing output keeps the
    // generated shape, so a perturbed input makes either the inputs or the
    // output disagree -- the plan must then throw
    bool expect_throw = false;
    if (!all_scalar_inputs) {
      size_t r = 0;
      for (int k = 1; k <= nin; ++k)
        if (!ops[k].scalar) r = std::max(r, ops[k].sizes.size());
      std::vector<int64_t> b(r, 1);
      for (int k = 1; k <= nin; ++k) {
        if (ops[k].scalar) continue;
        const size_t off = r - ops[k].sizes.size();
        for (size_t i = 0; i < ops[k].sizes.size(); ++i) {
          const int64_t v = ops[k].sizes[i];
          if (v == 1 || v == b[off + i]) continue;
          if (b[off + i] == 1) b[off + i] = v;
          else expect_throw = true;
        }
      }
      if (!new_out) expect_throw = expect_throw || b != shape;
      if (!expect_throw) {
        // every input's strides on the (possibly lower-rank) broadcast shape
        shape = b;
        full.assign(1 + nin, std::vector<int64_t>(r, 0));
        for (int k = 1; k <= nin; ++k) {
          if (ops[k].scalar) continue;
          const size_t off = r - ops[k].sizes.size();
          for (size_t i = 0; i < ops[k].sizes.size(); ++i)
            full[k][off + i] = (ops[k].sizes[i] == 1 && b[off + i] != 1) ? 0 : ops[k].strides[i];
        }
      }
    }
    total = 1;
    for (int64_t v : shape) total *= v;
    if (!new_out) {
      ops[0].sizes = shape;
      dense_perm(shape, ops[0].strides);
      full[0] = ops[0].strides;
    }
    supa::Plan p;
    try {
      p = supa::make_plan(ops);
    } catch (const std::invalid_argument&) {
      ++throws;
      if (!expect_throw) {
        std::printf("FAIL case %d: unexpected throw\n", it);
        return 1;
      }
      continue;
    }
    if (expect_throw) {
      std::printf("FAIL case %d: mismatched shapes accepted\n", it);
      return 1;
    }
    if (all_scalar_inputs) shape = ops[0].sizes;
    if (p.shape != shape) {
      std::printf("FAIL case %d: broadcast shape\n", it);
      return 1;
    }
    if (new_out) {
      full[0] = p.out_strides[0];
      // dense: over the dims of size > 1 sorted by stride, each stride is the
      // product of the sizes of the faster dims
      std::vector<std::pair<int64_t, int64_t>> sd;
      for (size_t i = 0; i < shape.size(); ++i)
        if (shape[i] > 1) sd.push_back({p.out_strides[0][i], shape[i]});
      std::sort(sd.begin(), sd.end());
      bool dense = true;
      int64_t want = 1;
      for (const auto& q : sd) {
        dense = dense && q.first == want;
        want *= q.second;
      }
      if (total > 0 && !dense) {
        std::printf("FAIL case %d: new output strides are not dense\n", it);
        return 1;
      }
    }
    for (int k = 1; k <= nin; ++k)
      if (ops[k].scalar) std::fill(full[k].begin(), full[k].end(), 0);
    std::vector<Tuple> want, got;
    visit_logical(shape, full, want);
    visit_plan(p, 1 + nin, got);
    std::sort(want.begin(), want.end());
    std::sort(got.begin(), got.end());
    if (want != got) {
      std::printf("FAIL case %d: plan visits %zu tuples, expected %zu\n", it, got.size(), want.size());
      return 1;
    }
    ++plans;
  }
  std::printf("OK %ld plans checked, %ld mismatches rejected\n", plans, throws);
  return 0;
}
