"""CPU checks of the in-chunk profile's matching of profiler dispatches to
the libsvla calls of a chunk (smolvla.census), on synthetic profiler rows."""

import pytest

from smolvla import census


def row(name, t0, t1, did=0):
    return {"Kernel_Name": name, "Start_Timestamp": str(t0), "End_Timestamp": str(t1),
            "Dispatch_Id": str(did)}


CALLS = [("svla_rmsnorm_bf16", "hbm", 0, 100, "rmsnorm 4x8"),
         ("svla_linear_bf16", "mfma", 2000, 300, "linear 4x8x8"),
         ("svla_expert_run", "hbm", 5000, 900, "fused action expert"),
         ("svla_linear_bf16", "mfma", 2000, 300, "linear 4x8x8")]


def chunk(t):
    return [row("void (anonymous namespace)::rmsnorm_kernel(a)", t, t + 2),
            row("void at::native::(anonymous namespace)::copy_kernel(b)", t + 2, t + 3),
            row("void (anonymous namespace)::gemm_line_kernel<64, 64>(GemmArgs)", t + 3, t + 9),
            row("void (anonymous namespace)::clear_u32_kernel(unsigned*, long)", t + 9, t + 10),
            row("void (anonymous namespace)::expert_kernel(XArgs)", t + 10, t + 60),
            row("__amd_rocclr_copyBuffer", t + 60, t + 61),
            row("void (anonymous namespace)::skinny_kernel<16>(GemmArgs)", t + 61, t + 64)]


def test_own_dispatches_keep_only_the_library_kernels():
    own = census.own_dispatches(chunk(0))
    assert [census.short_kernel_name(r["Kernel_Name"]) for r in own] == [
        "rmsnorm_kernel", "gemm_line_kernel<64, 64>", "clear_u32_kernel", "expert_kernel",
        "skinny_kernel<16>"]


def test_last_chunk_is_matched_call_by_call():
    rows = chunk(0) + chunk(100)
    al = census.align_last_chunk(CALLS, census.own_dispatches(rows))
    assert [i for i, _ in al] == [0, 1, 2, 2, 3]
    assert int(al[0][1]["Start_Timestamp"]) == 100          # the last chunk, not the first
    table, total_ms, n = census.profile_table(CALLS, {"rmsnorm 4x8": 1.0}, rows, [], 1)
    assert n == 5 and "fused action expert" in table
    assert abs(total_ms - (2 + 6 + 1 + 50 + 3) * 1e-6) < 1e-12     # ns -> ms


def test_a_kernel_of_the_wrong_family_is_refused():
    rows = chunk(0)
    rows[2] = row("void (anonymous namespace)::attention_kernel<true, 1>(AttnArgs)", 3, 9)
    with pytest.raises(ValueError, match="expects"):
        census.align_last_chunk(CALLS, census.own_dispatches(rows))
