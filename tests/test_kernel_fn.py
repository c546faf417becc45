"""kernel_fn handling on the CPU (attention.py:12-50): the reference's
use_custom_einsum switch exists and runs, default_kernel / threshold_kernel
map to their softmax scales, user kernels of the form exp(s q.k + c) are
probed for s (the reference test's exp(q.k / (2 sqrt(d))),
test_mapped_attention.py:1122-1144, gives 1 / (2 sqrt(d))), and kernels of any
other form raise NotImplementedError before anything reaches the GPU."""
import math

import numpy as np
import pytest
import torch

import jaxmodules_amd as jm
from jaxmodules_amd import attention as A


def test_use_custom_einsum_is_importable_and_runs():
    from jaxmodules_amd.attention import use_custom_einsum

    assert use_custom_einsum() is None
    assert jm.use_custom_einsum is use_custom_einsum


@pytest.mark.parametrize("d", [16, 64, 128])
def test_builtin_kernel_scales(d):
    assert A.kernel_scale(A.default_kernel, d) == pytest.approx(1 / math.sqrt(d))
    assert A.kernel_scale(A.threshold_kernel(2.5), d) == 1.0
    assert A.kernel_scale(A.threshold_kernel(), d) == 1.0


@pytest.mark.parametrize("d", [16, 48, 128])
def test_probe_reference_custom_kernel(d):
    def custom_kernel(q, k):  # the reference test's kernel, with numpy in place of jnp
        return np.exp(np.dot(q, k) / (2 * np.sqrt(k.shape[-1])))

    assert A.kernel_scale(custom_kernel, d) == pytest.approx(1 / (2 * math.sqrt(d)), rel=1e-6)


def test_probe_affine_log_kernels():
    assert A.kernel_scale(lambda q, k: np.exp(0.3 * np.dot(q, k) - 1.2), 32) == pytest.approx(0.3, rel=1e-6)
    assert A.kernel_scale(lambda q, k: 7.0 * np.exp(-0.5 * np.dot(q, k)), 32) == pytest.approx(-0.5, rel=1e-6)
    assert A.kernel_scale(lambda q, k: np.exp(0 * np.dot(q, k)), 32) == 0.0
    # a kernel written with torch operations (numpy input rejected) is probed through tensors
    def torch_kernel(q, k):
        if not isinstance(q, torch.Tensor):
            raise TypeError("tensors only")
        return torch.exp(torch.dot(q, k) / 4)
    assert A.kernel_scale(torch_kernel, 16) == pytest.approx(0.25, rel=1e-6)


@pytest.mark.parametrize("fn", [
    lambda q, k: np.maximum(np.dot(q, k), 0) + 1e-3,       # not an exponential
    lambda q, k: np.exp(np.dot(q, k) ** 2),                 # not affine in q.k
    lambda q, k: np.exp(np.dot(q, q) + np.dot(q, k)),       # depends on |q| too
    lambda q, k: -np.exp(np.dot(q, k)),                     # negative scores
])
def test_probe_rejects_other_kernels(fn):
    with pytest.raises(NotImplementedError):
        A.kernel_scale(fn, 32)


def test_rejected_kernel_raises_before_gpu():
    Q = torch.zeros(8, 2, 16)
    with pytest.raises(NotImplementedError):
        jm.masked_attention_via_map(Q, Q, Q, kernel_fn=lambda q, k: np.dot(q, k) ** 2 + 1)


def test_head_dims_up_to_512():
    """The host pads d to the next kernel head dimension, 64, 128, 256 or 512;
    beyond 512 it raises NotImplementedError before any GPU work."""
    from jaxmodules_amd import attention as A

    assert [A._kernel_dim(d) for d in (1, 64, 65, 128, 129, 256, 257, 512)] == [64, 64, 128, 128, 256, 256,
                                                                               512, 512]
    with pytest.raises(NotImplementedError):
        A._kernel_dim(513)
