"""The reference test program's parameter matrix (tests/test_main.cpp:145-161), shared by the CPU and GPU
parity tests."""


def reference_cases():
    """4 distributions x degree {1,4,8,16} x RHS {8,16,32,64} on a 9 x 17 block grid; seeds 11.. in order;
    local columns iff the seed is odd.  Returns (distribution, degree, rhs, locality, seed) tuples."""
    cases = []
    seed = 11
    for distribution in ("uniform", "low", "high", "bimodal"):
        for degree in (1, 4, 8, 16):
            for rhs in (8, 16, 32, 64):
                cases.append((distribution, degree, rhs, "local" if seed & 1 else "random", seed))
                seed += 1
    return cases
