"""GPU: the launcher paths that hip_attn_set_option selects, each against the CPU oracle.

- LLMGEN_OPT_DECODE_MERGE_KERNEL = 1: split-K partials merged by the separate merge kernel (the path that
  launches with more than 2^18 (sequence, KV head) pairs take) instead of inside the decode kernel;
- LLMGEN_OPT_DECODE_ROW_WAVES = 8: 8-wave workgroups for the decode rows of mixed steps;
- LLMGEN_OPT_ATTN_PART_MIN (the reference's SV_ATTN_PART, attention.cu:219-229): longer split-K parts, down to
  one part per sequence.
Every option is restored after its test.
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest

from harness import compare, run_gpu, run_oracle
from llmgen_amd._lib import lib
from llmgen_amd.workloads import make, to_u16

pytestmark = pytest.mark.gpu

OPT_ATTN_PART_MIN, OPT_DECODE_ROW_WAVES, OPT_DECODE_MERGE_KERNEL = 0, 1, 2


@contextlib.contextmanager
def option(which, value):
    prev = lib().hip_attn_set_option(which, value)
    assert prev >= 0, f"option {which}={value} refused"
    try:
        yield
    finally:
        assert lib().hip_attn_set_option(which, prev) == value


def _check(name, sampled=False):
    wl = make(name)
    t = wl.tensors(device="cuda")
    out, _, _ = run_gpu(wl, t)
    if sampled:
        from test_gpu_attention import _sample_rows

        rows = _sample_rows(wl, wl.meta(64))
        _, _, _, of = run_oracle(wl, t, rows=rows, threads=16)
        compare(to_u16(out)[rows], of, name)
    else:
        _, _, _, of = run_oracle(wl, t)
        compare(to_u16(out), of, name)
    return to_u16(out)


@pytest.mark.parametrize("name", ["c1", "kt_decode", "gqa8d", "gqa16d", "bs6d", "c5d"])
def test_separate_merge_kernel(gpu, name):
    print(f"[gpu-test] merge kernel {name}", flush=True)
    with option(OPT_DECODE_MERGE_KERNEL, 1):
        _check(name, sampled=name == "c5d")


@pytest.mark.parametrize("name", ["cpu_mixed", "gqa8", "bs6", "c4"])
def test_eight_wave_decode_rows(gpu, name):
    print(f"[gpu-test] 8-wave decode rows {name}", flush=True)
    with option(OPT_DECODE_ROW_WAVES, 8):
        _check(name, sampled=name == "c4")


@pytest.mark.parametrize("part_min", [256, 100000])
@pytest.mark.parametrize("name", ["c1", "kt_decode", "c2"])
def test_attn_part_min(gpu, name, part_min):
    print(f"[gpu-test] SV_ATTN_PART={part_min} {name}", flush=True)
    with option(OPT_ATTN_PART_MIN, part_min):
        _check(name)


def test_option_rejects_bad_values(gpu):
    L = lib()
    assert L.hip_attn_set_option(7, 1) == -1
    assert L.hip_attn_set_option(OPT_DECODE_ROW_WAVES, 6) == -1
    assert L.hip_attn_set_option(OPT_ATTN_PART_MIN, -5) == -1
