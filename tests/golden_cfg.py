"""KV-cache fixture configurations shared by tests/golden/make_golden.py and
the tests: (layers, heads, head_dim, sink, window, pool_block, max_context,
number of stored positions)."""
KV_CFGS = {
    "t": (2, 2, 4, 2, 16, 4, 128, 40),
    "p": (1, 2, 32, 4, 24, 5, 400, 150),
    "s": (1, 1, 16, 10, 12, 3, 60, 70),
}
