// Iteration planner for elementwise ops: broadcast, output layout, dimension
// order and coalescing.  Plain C++ (no torch, no HIP) so it is testable on a
// machine without a GPU.
//
// It plays the role upstream TensorIteratorBase plays for the reference's
// gpu_kernel (torch_supa/csrc/aten/ops/kernels/elementwise/Loops.cuh:110-134,
// CUDALoops.cuh:857-937).  The output-layout rule is the one a user can
// observe, so it follows upstream exactly: dimensions are ordered by the
// strides of the operands (outputs first, then inputs), a broadcast stride
// never decides, ties on equal strides put the smaller dimension first, and a
// new output is dense in that order (so a permuted dense input yields an
// output with the same permutation).  Coalescing is internal.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace supa {

struct PlanOperand {
  std::vector<int64_t> sizes;    // tensor order (dim 0 = outermost)
  std::vector<int64_t> strides;  // elements, tensor order
  bool is_output = false;
  bool allocate = false;  // output to be created (sizes/strides ignored) or resized
  bool scalar = false;    // immediate scalar: no shape, no strides
};

struct Plan {
  std::vector<int64_t> shape;                     // broadcast shape, tensor order
  std::vector<std::vector<int64_t>> out_strides;  // per operand; filled for outputs with allocate=true
  // Iteration space for the kernels: dims fastest-first after reordering and
  // coalescing; strides per operand in elements (0 for scalars).
  std::vector<int64_t> it_sizes;
  std::vector<std::vector<int64_t>> it_strides;
  int64_t numel = 1;
};

// Broadcast shape of the non-scalar input operands (outputs do not take part,
// as with TensorIterator's resize_outputs; with no tensor input the first
// existing output gives the shape).  Throws std::invalid_argument on a
// mismatch.
std::vector<int64_t> broadcast_shape(const std::vector<PlanOperand>& ops);

// Full plan.  Outputs with allocate=false must already have `shape`.
Plan make_plan(const std::vector<PlanOperand>& ops);

// Contiguous strides of a shape (tensor order).
std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape);

}  // namespace supa
