"""Shared checks for the paged KV cache (oracle and GPU)."""

import numpy as np


def check_allocator_invariants(tables, refcounts, free_list, max_pages):
    """Every page is either free (once) or referenced; a reference count equals the references from all tables."""
    references = np.zeros(max_pages, dtype=np.int64)
    for table in tables:
        mapped = table[table >= 0]
        assert len(set(mapped.tolist())) == mapped.size, "a slot maps one page twice"
        np.add.at(references, mapped, 1)
    assert np.array_equal(references, refcounts), "reference counts differ from table references"
    free = np.asarray(free_list)
    assert len(set(free.tolist())) == free.size, "a page is free twice"
    assert np.all(refcounts[free] == 0), "a free page is referenced"
    assert free.size + np.count_nonzero(refcounts) == max_pages, "a page is neither free nor referenced"
