"""CPU oracle for the per-step sparse decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithm of each function on
the decode hot path of mini-hisparse.  It is the checker the HIP kernels are
compared against; it is never shipped and never measured as the product.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package (``mini_hisparse_amd``) never
imports it and fails loudly when its HIP library is missing.

Modules and the reference code each one follows (paths under the reference
checkout):

* ``resolver``  -- ``resolve_rows`` (``mini_hisparse/row_index.py:59-137``)
* ``quest``     -- ``quest_selection`` scores and per-head top-k
                   (``mini_hisparse/selection.py:80-101``), ``Selection``
                   canonicalisation (``selection.py:18-64``)
* ``union``     -- ``LogicalTopK.from_selection`` (``row_index.py:20-31``)
* ``gather``    -- the CPU row gather loop (``mini_hisparse/hybrid.py:466-472``)
* ``append``    -- the single-token append: pool rows, Quest bounds, host
                   mirror (``mini_hisparse/storage.py:246-319``)
* ``attention`` -- the torch row attention (``mini_hisparse/attention.py:26-35``),
                   ``dense_attention`` (``selection.py:158-163``),
                   ``selection_oracle`` (``selection.py:104-126``) and the
                   paged layout's window state (``reference/kernels.py:12-68``)
* ``cpu_path``  -- the reference's CPU decode path of one (request, layer) as
                   torch CPU ops (Quest, union, resolver, per-row gather loop,
                   row attention): what ``bench.py``'s ``cpu_baseline`` leg
                   times, not a checker.

Pinning (what each function is checked against, besides the GPU):

* resolver  -- the reference's walkthrough vectors
  (``docs/reports/index-walkthrough.json``), the reference tests' known
  counts, reference-generated multi-step trajectories in
  ``tests/golden/``, an independent sequential formulation and invariants.
* quest     -- the reference's known answer (pages ``[0, 2]``), reference-
  generated selections in ``tests/golden/``, exact rational brute force on
  tiny inputs, and the special cases (``top >= count``, forced pages).
* union     -- reference-generated vectors and an independent formulation.
* gather    -- byte equality of copied rows with the host rows.
* append    -- known answers of torch's NaN / signed-zero rule, equality with
  ``numpy.minimum``/``maximum`` where that rule and numpy's agree (no NaN, no
  equal zeros), a page filled row by row equals its exact column extrema, and
  (on the GPU) equality with ``torch.minimum``/``torch.maximum`` themselves.
* attention -- a scalar textbook softmax in float64 on small inputs, and the
  special cases (all masked -> 0, one row -> V, equal scores -> mean of V);
  window states merged across windows (the merge rule of
  ``reference/attention.py:11-18``) equal dense attention over the union of
  their tokens, and a head that reads nothing has (-inf, 0, 0).
"""

from .append import append_rows, append_tokens, bound_max, bound_min, takes_new_max, takes_new_min
from .attention import attend_rows, dense_attention, row_attention_rows, selection_oracle, window_state
from .gather import gather_rows
from .quest import quest_pages, quest_scores, quest_selection_positions
from .resolver import resolve_rows
from .union import from_selection

__all__ = [
    "append_rows",
    "append_tokens",
    "attend_rows",
    "bound_max",
    "bound_min",
    "takes_new_max",
    "takes_new_min",
    "dense_attention",
    "from_selection",
    "gather_rows",
    "quest_pages",
    "quest_scores",
    "quest_selection_positions",
    "resolve_rows",
    "row_attention_rows",
    "selection_oracle",
    "window_state",
]
