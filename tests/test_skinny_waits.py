"""The skinny kernel's counted waits (csrc/nb_gemv_skinny.hip, `after`),
checked on the CPU against a model of each wave's vector-memory issue order.

A wave issues, before its loop, the x slices X(0 .. kLead - 1) (two loads
each) and then the weight slots W(0 .. depth - 1) (five loads each); item
i's step then waits, reads its slot, issues X(g + kLead) if i is the first
of the R items of slice g = i / R, computes, and issues W(i + depth).
Loads complete in issue order, so the wait `s_waitcnt vmcnt(after(i))` is
right when after(i) is exactly the number of loads issued after the later
of W(i) and (first item of a slice) X(g).  `kernel_after` restates the
kernel's formula; `simulate` derives the count from the issue sequence.
A formula that waited too little would read a slot or an x buffer before
its bytes arrive; one that waited too much would only be slower -- both
fail here.
"""
import pytest


def kernel_after(i, R, depth, lead, nitems):
    nslices = nitems // R

    def x_at(j):
        return 2 if (j % R == 0 and j // R + lead < nslices) else 0

    def w_at(j):
        return 5 if j + depth < nitems else 0

    nw = 0
    if i < depth:
        nw += 5 * len(range(i + 1, min(depth, nitems)))
        nw += sum(x_at(j) + w_at(j) for j in range(i))
    else:
        nw += sum(x_at(j) + w_at(j) for j in range(i - depth + 1, i))
    if i % R:
        return nw
    g = i // R
    if g < lead:
        nx = 2 * len(range(g + 1, min(lead, nslices))) + 5 * min(depth, nitems)
        nx += sum(x_at(j) + w_at(j) for j in range(i))
    else:
        j0 = (g - lead) * R
        nx = w_at(j0) + sum(x_at(j) + w_at(j) for j in range(j0 + 1, i))
    return min(nw, nx)


def simulate(R, depth, lead, nitems):
    nslices = nitems // R
    seq = []
    for g in range(min(lead, nslices)):
        seq += [("X", g)] * 2
    for d in range(min(depth, nitems)):
        seq += [("W", d)] * 5
    counts = []
    for i in range(nitems):
        g = i // R
        need = [("W", i)] + ([("X", g)] if i % R == 0 else [])
        last = max(max(k for k, e in enumerate(seq) if e == n) for n in need)
        counts.append(len(seq) - 1 - last)
        if i % R == 0 and g + lead < nslices:
            seq += [("X", g + lead)] * 2
        if i + depth < nitems:
            seq += [("W", i + depth)] * 5
    return counts


@pytest.mark.parametrize("R", [1, 2, 3, 4])
@pytest.mark.parametrize("depth,lead", [(2, 1), (3, 1), (3, 2)])
def test_wait_counts_follow_the_issue_order(R, depth, lead):
    for ns in range(1, 40):
        n = ns * R
        want = simulate(R, depth, lead, n)
        got = [kernel_after(i, R, depth, lead, n) for i in range(n)]
        assert got == want, (R, depth, lead, n)


def test_steady_state_counts_fit_the_immediate_forms():
    """wait_vm_n has immediate forms for 1..24 (anything else waits for all
    loads, always enough); in the loop's steady state the counts stay
    within them."""
    worst = max(kernel_after(i, R, 3, lead, n)
                for R in (1, 2) for lead in (1, 2) for n in range(2, 200, 2)
                for i in range(3, n))
    assert worst <= 24


def test_the_kernel_uses_these_parameters():
    """The launch configurations the formula is checked for: three ring
    slots per wave, x one or two slices ahead (two or three buffers), two
    128-row parts per slice on the tile layout, one on the reference one."""
    import os
    src = open(os.path.join(os.path.dirname(__file__), "..", "nativebit_amd", "csrc",
                            "nb_gemv_skinny.hip")).read()
    assert "#define NB_SK_DEPTH 3" in src
    assert "constexpr int kLead = NXB - 1;" in src
    assert "return tile ? 2 : 1;" in src
    assert "? 3 : 2;" in src  # skinny_xbufs: three x buffers where they fit, else two
