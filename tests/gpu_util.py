"""Helpers shared by the GPU parity tests: run the HIP kernels through the
drop-in binding and evaluate the CPU oracle on the same inputs."""
import sys

import numpy as np
import torch

from gdn_kernel_amd import binding
from gdn_kernel_amd.workloads import to_numpy
from oracle import gdn_oracle as O

# Tolerances of this path: bf16 output within atol/rtol 1e-2; fp32 state within
# rtol 1e-3 (atol 1e-5 covers elements that cancel to ~0).
OUT_RTOL = OUT_ATOL = 1e-2
STATE_RTOL, STATE_ATOL = 1e-3, 1e-5


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_decode(w, device, in_place=True, state=None):
    """Run the decode kernel; returns (output, new_state) on the device."""
    d = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    st = d["state"] if state is None else state
    out = torch.full_like(d["v"], float("nan"))
    if st is None:
        ns = torch.full((d["q"].shape[0], d["v"].shape[2], 128, 128), float("nan"),
                        device=device, dtype=torch.float32)
    elif in_place:
        ns = st
    else:
        ns = torch.full_like(st, float("nan"))
    binding.decode_kernel(d["q"], d["k"], d["v"], st, d["A_log"], d["a"], d["dt_bias"], d["b"],
                          d["scale"], out, ns)
    return out, ns


def oracle_decode(w):
    return O.decode(to_numpy(w["q"]), to_numpy(w["k"]), to_numpy(w["v"]), to_numpy(w["state"]),
                    to_numpy(w["A_log"]), to_numpy(w["a"]), to_numpy(w["dt_bias"]),
                    to_numpy(w["b"]), w["scale"])


def run_prefill(p, device, in_place=False):
    d = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    T, Hv = d["v"].shape[0], d["v"].shape[1]
    N = d["cu_seqlens"].numel() - 1
    out = torch.full((T, Hv, 128), float("nan"), device=device, dtype=torch.bfloat16)
    if in_place and d["state"] is not None:
        ns = d["state"]
    else:
        ns = torch.full((N, Hv, 128, 128), float("nan"), device=device, dtype=torch.float32)
    binding.prefill_kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"],
                           d["b"], d["cu_seqlens"], d["scale"], out, ns)
    return out, ns


def oracle_prefill(p, chunked=True):
    fn = O.prefill_chunked if chunked else O.prefill_sequential
    return fn(to_numpy(p["q"]), to_numpy(p["k"]), to_numpy(p["v"]), to_numpy(p["state"]),
              to_numpy(p["A_log"]), to_numpy(p["a"]), to_numpy(p["dt_bias"]), to_numpy(p["b"]),
              p["cu_seqlens"].cpu().numpy(), p["scale"])


def host(t):
    return t.detach().cpu().double().numpy()
