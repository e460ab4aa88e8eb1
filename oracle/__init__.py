"""CPU oracle for the render pipeline: TEST INFRASTRUCTURE, never part of the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the reference that the HIP backend is compared against (and,
in ``bench.py``, as the reported CPU baseline). ``diffrast_amd`` never imports it and has no
CPU fallback.

``oracle.reference`` restates the pure-PyTorch reference backend of diffrast
(``src/diffrast/backends/reference.py``) and ``oracle.cube`` its cube-map geometry
(``src/diffrast/backends/_cube.py``). The visibility arithmetic keeps the reference's floating
point operations one for one, so that on the same CPU both pick the same triangle for every
pixel. Every function cites the reference lines it follows.

How each function is pinned (the tests named are under ``tests/``):

* visibility, fill rule, area tolerance, culling, depth layers — integer-exact owners, the
  screen-space float64 rasterizer, closed fans, sliver areas and clip-scale invariance
  (``test_oracle_raster.py``), plus golden vectors written by the reference itself
  (``tests/golden/``).
* ``rasterize_from_ids`` — float64 closed forms and finite differences of ``rast_db``.
* ``interpolate`` — vertex identity, exact affine derivatives at ``w = 1``.
* texture sampling and the mip chain — texel-centre identities, wrap/clamp/zero closed forms,
  Fraction-exact area weights, block means and golden vectors.
* cube maps — a brute-force float64 OpenGL sampler that finds neighbouring texels by
  projection, and golden vectors.
* antialias — exact straight and slanted edge areas, edge-length gradients, finite
  differences, and golden vectors.
* edge adjacency and silhouettes — hand-built meshes and golden vectors.

``log2`` rounding of the level of detail is not pinned beyond the 1e-5 tolerance: the reference
takes it from ``torch.log2``, whose ulp behaviour is PyTorch's.
"""
