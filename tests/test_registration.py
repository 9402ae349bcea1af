"""Registration hygiene of the PrivateUse1 backend, as the reference checks
its own (test/test_dispatch_registration.py:13-17): after loading the
backend no operator has a kernel registered without a schema (a "dangling"
impl, e.g. a misspelt overload name), and the path's operators do have
PrivateUse1 kernels."""
import pytest
import torch

torch_supa = pytest.importorskip("torch_supa")


def test_no_dangling_impls():
    assert torch._C._dispatch_find_dangling_impls() == []


@pytest.mark.parametrize("op", [
    "aten::add.out", "aten::mul.out", "aten::div.out", "aten::gelu.out", "aten::gelu_backward.grad_input",
    "aten::silu.out", "aten::sigmoid.out", "aten::_log_softmax.out", "aten::_log_softmax_backward_data.out",
    "aten::nll_loss_forward.output", "aten::nll_loss_backward.grad_input", "aten::mse_loss.out",
    "aten::smooth_l1_loss.out", "aten::binary_cross_entropy_with_logits", "aten::sum.IntList_out",
    "aten::_foreach_add_.List", "aten::_foreach_mul_.Scalar", "aten::_fused_adamw_", "aten::_copy_from",
    "aten::fill_.Scalar", "aten::cross_entropy_loss",
])
def test_path_ops_have_privateuse1_kernels(op):
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op, "PrivateUse1"), op
