"""The old cache's one-pass layout and address read before the shift-cache build
(_kvr_layout.kv_layers, C++ on torch's tensor metadata) against the per-tensor
Python reads it replaces, and build_halo_cache's layout checks through it: the
same acceptance and the same errors as the per-tensor checks."""

from __future__ import annotations

import ctypes
import struct

import pytest
import torch

from kv_cache_repair_amd import cache as C
from kv_cache_repair_amd.kernels.executor import _validate_cache, tensor_layout, uniform_layers


def kv_layers(layers):
    return tensor_layout().kv_layers(layers)


def addresses(raw: bytes) -> list[int]:
    return list(struct.unpack(f"{len(raw) // 8}Q", raw))


def cache_of(pairs):
    return C.cache_from_tensors(pairs)


def uniform_pairs(layers=5, heads=2, tokens=7, dim=8, dtype=torch.bfloat16):
    return [(torch.randn(1, heads, tokens, dim).to(dtype), torch.randn(1, heads, tokens, dim).to(dtype))
            for _ in range(layers)]


def test_uniform_cache_gives_every_address_in_layer_order():
    pairs = uniform_pairs()
    k_raw, v_raw, first, uniform = kv_layers(cache_of(pairs).layers)
    assert uniform is True and first is pairs[0][0]
    assert addresses(k_raw) == [k.data_ptr() for k, _ in pairs]
    assert addresses(v_raw) == [v.data_ptr() for _, v in pairs]


def test_views_into_one_slab_are_uniform():
    slab = torch.zeros(3, 2, 1, 2, 5, 8, dtype=torch.float16)
    views = slab.view(6, 1, 2, 5, 8).unbind(0)
    k_raw, v_raw, _, uniform = kv_layers(cache_of(zip(views[0::2], views[1::2])).layers)
    assert uniform is True
    assert addresses(k_raw) == [t.data_ptr() for t in views[0::2]]
    assert addresses(v_raw) == [t.data_ptr() for t in views[1::2]]


@pytest.mark.parametrize("change", ["strides", "dtype", "shape", "value_shape", "none", "meta"])
def test_any_layer_off_the_first_layout_is_not_uniform(change):
    pairs = uniform_pairs()
    k, v = pairs[3]
    if change == "strides":  # same shape, other strides
        k = torch.randn(1, 7, 2, 8).to(k.dtype).transpose(1, 2)
    elif change == "dtype":
        k = k.float()
    elif change == "shape":
        k = torch.randn(1, 2, 6, 8).to(k.dtype)
    elif change == "value_shape":
        v = torch.randn(1, 2, 7, 4).to(v.dtype)
    elif change == "none":
        v = None
    else:
        k = torch.empty(k.shape, dtype=k.dtype, device="meta")
    pairs[3] = (k, v)
    k_raw, v_raw, first, uniform = kv_layers(cache_of(pairs).layers)
    assert uniform is False and k_raw == b"" and v_raw == b"" and first is pairs[0][0]


def test_empty_and_malformed_layer_lists():
    assert kv_layers([]) == (b"", b"", None, False)

    class NoValues:
        keys = torch.zeros(1)

    with pytest.raises(AttributeError):
        kv_layers([NoValues()])
    with pytest.raises(TypeError):
        kv_layers(3)


def test_layer_addresses_refuse_what_the_per_tensor_checks_refuse():
    # CPU tensors: uniform, but not on a ROCm GPU -> the device error of the checks
    pairs = uniform_pairs()
    with pytest.raises(ValueError, match="ROCm GPU device"):
        C._layer_addresses(cache_of(pairs), "build_halo_cache")
    with pytest.raises(ValueError, match="ROCm GPU device"):
        C._check_uniform(pairs, "build_halo_cache")
    # not uniform: the per-tensor path names the problem, as before
    bad = list(pairs)
    bad[2] = (bad[2][0].float(), bad[2][1])
    with pytest.raises(ValueError, match="share dtype and device"):
        C._layer_addresses(cache_of(bad), "build_halo_cache")
    bad = list(pairs)
    bad[1] = (torch.randn(1, 2, 7, 4).to(torch.bfloat16), bad[1][1])
    with pytest.raises(ValueError, match="one geometry"):
        C._layer_addresses(cache_of(bad), "build_halo_cache")
    with pytest.raises(IndexError):
        C._layer_addresses(cache_of([]), "build_halo_cache")


def test_address_arrays_are_ctypes_pointer_arrays(monkeypatch):
    """On a uniform GPU layout the helper hands the launch ctypes arrays of the
    addresses (the device check is stubbed: no GPU here)."""
    pairs = uniform_pairs(layers=3)
    monkeypatch.setattr(torch.Tensor, "get_device", lambda self: 0)
    monkeypatch.setattr(C, "_require_device", lambda tensor, what: None)
    first, k_arr, v_arr = C._layer_addresses(cache_of(pairs), "build_halo_cache")
    assert first is pairs[0][0]
    assert isinstance(k_arr, ctypes.Array) and len(k_arr) == 3
    assert list(k_arr) == [k.data_ptr() for k, _ in pairs] and list(v_arr) == [v.data_ptr() for _, v in pairs]


def test_uniform_layers_is_none_off_one_layout_or_without_kv_attributes():
    pairs = uniform_pairs(layers=3)
    k_raw, v_raw, first = uniform_layers(cache_of(pairs).layers)
    assert first is pairs[0][0] and addresses(k_raw) == [k.data_ptr() for k, _ in pairs]
    pairs[1] = (pairs[1][0].float(), pairs[1][1])
    assert uniform_layers(cache_of(pairs).layers) is None

    class NoKeys:
        values = torch.zeros(1)

    assert uniform_layers([NoKeys()]) is None


def test_validate_cache_fast_path_accepts_and_refuses_as_the_per_layer_checks(monkeypatch):
    pairs = uniform_pairs(layers=4, tokens=7)
    # CPU caches take the per-layer checks (no device check there)
    assert _validate_cache(cache_of(pairs), 7) == 4
    with pytest.raises(ValueError, match="single-batch edited token length"):
        _validate_cache(cache_of(pairs), 6)
    # as on a GPU: the one-pass fast path; a wrong length still reaches the named check
    monkeypatch.setattr(torch.Tensor, "get_device", lambda self: 0)
    assert _validate_cache(cache_of(pairs), 7) == 4
    with pytest.raises(ValueError, match="single-batch edited token length"):
        _validate_cache(cache_of(pairs), 6)
    pairs[2] = (pairs[2][0], pairs[2][1].float())
    with pytest.raises(ValueError, match="geometry, dtype, and device must agree"):
        _validate_cache(cache_of(pairs), 7)


def test_data_ptr_builtin_equals_the_tensor_method():
    """The module walk's address reader (a builtin of the layout extension)
    gives what torch.Tensor.data_ptr gives, for every kind of tensor a model
    holds, and refuses anything else."""
    data_ptr = tensor_layout().data_ptr
    base = torch.randn(6, 8)
    cases = [base, base[2:], base.t(), base[:, 3], torch.empty(0), torch.nn.Parameter(torch.zeros(3)),
             torch.zeros(2, 2, dtype=torch.bfloat16), torch.empty(4, device="meta")]
    for t in cases:
        assert data_ptr(t) == torch.Tensor.data_ptr(t)
    for bad in (None, 3, [base]):
        with pytest.raises(TypeError, match="expected a tensor"):
            data_ptr(bad)
