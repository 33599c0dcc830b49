"""CPU oracle for the GLiNER-Decide DeBERTa-v3 fused layer path.

TEST INFRASTRUCTURE ONLY. This package is the checker: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it.  The product path (the HIP library and its host mirror) never imports,
calls or falls back to anything in here.

`oracle.deberta` restates the reference graph in numpy (float64 arithmetic,
optionally rounded to fp16 at the reference's op boundaries); every function
cites the reference file:line it follows.  How each function is pinned is
listed in its docstring ("pinned by").
"""

from . import deberta  # noqa: F401
