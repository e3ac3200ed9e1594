"""CPU row gather (test infrastructure only).

Restates the CPU branch of ``HybridKVCache.resolve`` (``mini_hisparse/hybrid.py:466-472``)
and the index math of the Triton ``_gather`` (``row_kernels.py:46-55``): for each plan
entry with host row ``h >= 0`` (and device row ``d >= 0``), copy K and V of host row
``h`` into pool row ``d``.  Both pools are ``[blocks, 2, P, Hkv, D]``.
"""

from __future__ import annotations


def gather_rows(host, pool, miss_host_rows, miss_device_rows, page_size):
    """Copy in place into ``pool`` (numpy arrays or CPU torch tensors)."""
    hosts = [int(x) for x in list(miss_host_rows)]
    devices = [int(x) for x in list(miss_device_rows)]
    for h, d in zip(hosts, devices):
        if h >= 0 and d >= 0:
            hb, ho = divmod(h, page_size)
            db, do = divmod(d, page_size)
            pool[db, :, do] = host[hb, :, ho]
    return pool
