"""The allocation-free commitment uwc_b3_root_and_seed_static, through the C-ABI, against the
scratch-buffer entry point uwc_b3_root_and_seed on the same inputs: two calls in a row, the second
with a smaller input of another tree shape, roots and salted seeds equal (and the first root equal
to the oracle's keyed BLAKE3); an input above the static workspace's maximum is rejected on the
host before any GPU work."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle as O


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def test_static_commitment_rejects_oversized_input():
    from uwc_amd import _lib
    L = _lib.lib()
    buf = (ctypes.c_uint8 * 1024)()
    key = (ctypes.c_uint32 * 8)()
    too_big = (1 << 30) + 1024
    rc = L.uwc_b3_root_and_seed_static(ctypes.addressof(buf), too_big, ctypes.addressof(key), None, None, 0, None,
                                       None, None)
    assert rc == -1
    assert b"exceed the static workspace" in L.uwc_last_error()


@pytest.mark.gpu
def test_static_commitment_equals_scratch_commitment(dev):
    from uwc_amd import _lib, ops
    L = _lib.lib()
    rng = np.random.default_rng(7)
    key_b, prefix_b = rng.bytes(32), rng.bytes(32)
    key, prefix, salt = ops.words(key_b, dev), ops.words(prefix_b, dev), ops.SALT_A.to(dev)
    for call, nchunks in enumerate((65537, 1000)):  # the second call is smaller, with another tree shape
        host = rng.integers(0, 256, size=nchunks * 1024, dtype=np.uint8)
        data = torch.from_numpy(host).to(dev)
        nbytes = data.numel()
        outs = {name: torch.full((8,), -1, dtype=torch.int32, device=dev) for name in ("r0", "s0", "r1", "s1")}
        scratch = torch.empty(L.uwc_b3_scratch_words(nbytes), dtype=torch.int32, device=dev)
        assert L.uwc_b3_root_and_seed(data.data_ptr(), nbytes, key.data_ptr(), prefix.data_ptr(), salt.data_ptr(),
                                      nchunks, outs["r0"].data_ptr(), outs["s0"].data_ptr(), scratch.data_ptr(),
                                      scratch.numel(), _stream()) == 0
        rc = L.uwc_b3_root_and_seed_static(data.data_ptr(), nbytes, key.data_ptr(), prefix.data_ptr(), salt.data_ptr(),
                                           nchunks, outs["r1"].data_ptr(), outs["s1"].data_ptr(), _stream())
        assert rc == 0, L.uwc_last_error()
        torch.cuda.synchronize()
        assert torch.equal(outs["r0"], outs["r1"]), call
        assert torch.equal(outs["s0"], outs["s1"]), call
        if call == 0:
            assert ops.words_to_bytes(outs["r1"]) == O.b3(host.tobytes(), key_b)
