"""The allocation-free entry point launch_sparse_mla_noalloc (static device
scratch instead of a workspace) against launch_sparse_mla with a caller
workspace, through the C ABI: two calls in a row, the second smaller, each
bit-identical to the allocating entry."""

import ctypes as ct

import numpy as np
import pytest
import torch

from oracle import sparse_reference as sr
from tests.sparse_helpers import call_args, call_kwargs, to_device

pytestmark = pytest.mark.gpu


def launch_pair(tensors, policy, device):
    """Runs both entries on the same inputs; returns (noalloc output, allocating output)."""
    from ascendflow_amd import _native
    from ascendflow_amd._tensors import stream_handle
    from ascendflow_amd.sparse_attention.attention import make_params

    lib = _native.library()
    kw = call_kwargs(policy)
    params = make_params(*(kw[k] for k in ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS",
                                           "WINDOW", "TOPK", "S", "BM")), kw["DTYPE"], kw["SCALE"])
    nbytes = ct.c_uint64(0)
    _native.check(lib.workspace_size_sparse_mla(ct.byref(nbytes), ct.byref(params)), "workspace_size_sparse_mla")
    assert 0 < nbytes.value <= _native.SCRATCH_BYTES
    pointers = [t.data_ptr() for t in call_args(tensors)]
    stream = stream_handle(device)
    tensors["attention_out"].fill_(float("nan"))
    _native.check(lib.launch_sparse_mla_noalloc(stream, *pointers, ct.byref(params)), "launch_sparse_mla_noalloc")
    torch.cuda.synchronize()
    static = tensors["attention_out"].clone()
    workspace = torch.full((nbytes.value,), 0xCD, dtype=torch.uint8, device=device)
    tensors["attention_out"].fill_(float("nan"))
    _native.check(lib.launch_sparse_mla(stream, *pointers, workspace.data_ptr(), ct.byref(params)), "launch_sparse_mla")
    torch.cuda.synchronize()
    return static, tensors["attention_out"].clone()


def test_noalloc_entry_matches_the_workspace_entry_on_two_calls(device):
    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy

    # Call 1: a 4096-token prefill over a 4K context, the plan + persistent
    # path (a 12.6 MB plan in the scratch).
    print("\n[noalloc] call 1: prefill T4096 ctx4096", flush=True)
    policy = measurement_policy(batch=1, query_tokens=4096, context=4096)
    inputs = make_inputs(policy, 4096, device=device)
    static, allocating = launch_pair(dict(inputs.tensors), policy, device)
    assert torch.isfinite(static.float()).all()
    assert torch.equal(static, allocating), "noalloc output differs from launch_sparse_mla (call 1)"
    del inputs
    # Call 2, smaller: B4 x T16, where each token is split into parts whose
    # records the merge kernel combines, all inside the same scratch that still
    # holds call 1's plan.
    print("[noalloc] call 2: B4 T16 mixed (split parts)", flush=True)
    policy = sr.default_policy(B=4, T=16, MAX_SEQ=4096, ORI_BLOCKS=64, CMP_BLOCKS=64)
    data = sr.inputs(policy, "mixed")
    tensors = to_device(data, policy, device)
    static, allocating = launch_pair(tensors, policy, device)
    assert torch.equal(static, allocating), "noalloc output differs from launch_sparse_mla (call 2)"
    ref = sr.oracle_fp32(data, policy)
    err = float(np.max(np.abs(static.float().cpu().numpy() - ref)))
    assert err <= 1e-2 * float(np.max(np.abs(ref))), f"noalloc output off the oracle by {err}"
