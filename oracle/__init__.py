"""TEST INFRASTRUCTURE ONLY - CPU oracle of the MegaGate -> MegaMoE forward path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import this
package; the product (``hyper_multicore_amd``) never does. It restates the reference algorithm:
``router_ref.c`` (the route, bit-exact target for the gfx950 router) and ``moe_oracle.py`` (the
projection, route metadata, stable permutation, MX quantisation, expert math and combine).
"""
