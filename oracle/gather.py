"""CPU row gather (test infrastructure only).

Restates the CPU branch of ``HybridKVCache.resolve`` (``mini_hisparse/hybrid.py:466-472``)
and the index math of the Triton ``_gather`` (``row_kernels.py:46-55``): for each plan
entry with host row ``h >= 0`` (and device row ``d >= 0``), copy K and V of host row
``h`` into pool row ``d``.  Both pools are ``[blocks, 2, P, Hkv, D]``.

The HIP gather also skips an entry whose host row is at or past the host pool's
rows or whose device row is at or past the device pool's (the reference masks
only ``-1``; a valid plan never holds such rows, so both rules agree on every
plan the resolver produces).  ``bounded=True`` applies that rule here.
"""

from __future__ import annotations


def gather_rows(host, pool, miss_host_rows, miss_device_rows, page_size, bounded=False):
    """Copy in place into ``pool`` (numpy arrays or CPU torch tensors)."""
    hosts = [int(x) for x in list(miss_host_rows)]
    devices = [int(x) for x in list(miss_device_rows)]
    host_rows = len(host) * page_size if bounded else float("inf")
    pool_rows = len(pool) * page_size if bounded else float("inf")
    for h, d in zip(hosts, devices):
        if 0 <= h < host_rows and 0 <= d < pool_rows:
            hb, ho = divmod(h, page_size)
            db, do = divmod(d, page_size)
            pool[db, :, do] = host[hb, :, ho]
    return pool
