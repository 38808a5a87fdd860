"""Split-K work lists: every request's keys are cut into chunks of `chunk`
rows (at least one chunk per request) and each (request, chunk) pair is one
work item per KV head.  Items are dispatched longest first so that the
short tail chunks of ragged requests fill the end of the grid (greedy
longest-processing-time order); the partial-result slot of an item stays
its request-major index, so the dispatch order does not affect results.
"""
from ._device import upload

DEFAULT_CHUNK = 1024


def chunk_items(lengths, chunk):
    """[(request, chunk_index)] for all items, longest chunk first (stable)."""
    items = []
    for r, n in enumerate(lengths):
        n = int(n)
        count = max(1, -(-n // chunk))
        for c in range(count):
            items.append((min(chunk, n - c * chunk) if n > 0 else 0, r, c))
    items.sort(key=lambda x: -x[0])
    return [(r, c) for _, r, c in items]


def chunk_bound(n_req, rows_bound, chunk):
    """Upper bound on the number of items for n_req requests totalling at
    most rows_bound key rows (the C ABI's grid bound)."""
    return -(-int(rows_bound) // chunk) + int(n_req)


def upload_items(items, device):
    """int32 [n_items * 2] device tensor via the pinned staging ring."""
    return upload(device, [x for rc in items for x in rc])
