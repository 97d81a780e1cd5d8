"""Host-side restatement of the data-parallel tile scheduler.

``get_pids`` mirrors kernels/gemm/utils/common.py:38-83 (the device function
is ``g9::tile_coords`` in csrc/g9_common.hpp): the workgroup id is remapped so
each of the ``num_xcds`` XCDs (which receive workgroups round-robin) owns one
contiguous run of tile ids, then a GROUP_SIZE_M swizzle walks each run
``group_size_m`` tile rows at a time, column-major inside a group.  Used by the
stream-K planner and the tests.
"""


def cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def get_pids(pid: int, M: int, N: int, BM: int, BN: int, GRID_MN: int, NUM_XCDS: int, GROUP_SIZE_M: int):
    num_pid_m = cdiv(M, BM)
    num_pid_n = cdiv(N, BN)
    if NUM_XCDS != 1:
        per_xcd = cdiv(GRID_MN, NUM_XCDS)
        tall = GRID_MN % NUM_XCDS
        tall = NUM_XCDS if tall == 0 else tall
        xcd = pid % NUM_XCDS
        local = pid // NUM_XCDS
        if xcd < tall:
            pid = xcd * per_xcd + local
        else:
            pid = tall * per_xcd + (xcd - tall) * (per_xcd - 1) + local
    if GROUP_SIZE_M == 1:
        return pid // num_pid_n, pid % num_pid_n
    in_group = GROUP_SIZE_M * num_pid_n
    gid = pid // in_group
    first_m = gid * GROUP_SIZE_M
    gsize = min(num_pid_m - first_m, GROUP_SIZE_M)
    r = pid % in_group
    return first_m + r % gsize, r // gsize
