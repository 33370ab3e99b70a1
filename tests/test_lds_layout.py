"""The LDS tile layout of the GEMMs (and of the pipelined attention's K chunks):
rows of CPR 16-byte chunks stored unpadded, chunk c of row r at slot
c ^ chunk_swizzle16<CPR>(r) (edgebert_amd/csrc/kernels.hpp).  A fragment read
has the 32 lanes of a half-wave read one chunk of 32 consecutive rows; a
ds_read_b128 is served 8 lanes (128 bytes) at a time, so it is free of bank
conflicts when every 8 consecutive lanes hit 8 different 16-byte bank groups.
Restated here on the CPU and checked for 32 and 64 four-byte banks."""
import pytest


def chunk_swizzle16(cpr: int, r: int) -> int:
    if cpr == 16:
        return r & 15
    if cpr == 8:
        return (r & 7) ^ ((r >> 3) & 1)
    assert cpr == 4
    return ((r >> 1) & 3) ^ ((r >> 3) & 1)


@pytest.mark.parametrize("cpr", [4, 8, 16])
def test_swizzle_is_a_permutation_of_each_row(cpr):
    for r in range(256):
        assert sorted(c ^ chunk_swizzle16(cpr, r) for c in range(cpr)) == list(range(cpr))


@pytest.mark.parametrize("banks", [32, 64])
@pytest.mark.parametrize("cpr", [4, 8, 16])
def test_fragment_reads_are_conflict_free(cpr, banks):
    groups = banks // 4                    # 16-byte bank groups
    row_bytes = cpr * 16
    for base in range(0, 256, 32):         # the 32-row blocks of a tile
        for c in range(cpr):               # the chunk a half-wave reads
            addrs = [(base + l) * row_bytes + 16 * (c ^ chunk_swizzle16(cpr, base + l)) for l in range(32)]
            for g in range(0, 32, 8):
                bank_groups = {(a // 16) % groups for a in addrs[g:g + 8]}
                assert len(bank_groups) == 8, (cpr, banks, base, c, g)


def test_unswizzled_rows_would_conflict():
    """The check has teeth: without the swizzle, 8 rows of one chunk share a bank group."""
    cpr, groups = 8, 16
    addrs = [l * cpr * 16 for l in range(8)]
    assert len({(a // 16) % groups for a in addrs}) < 8
