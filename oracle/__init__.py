"""Test infrastructure, not product code: the CPU restatement of the reference's
PyTorch attention / norm / RoPE / KV-cache paths that the HIP kernels are checked
against (see ``oracle.ref``). Only tests, ``__graft_entry__.smoke`` and ``bench.py``'s
CPU-baseline leg may import it."""
