"""CPU oracle for the FP8 mixture-of-experts grouped-GEMM path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
pybind11 module, the ``hkmoe`` host package) imports, links or executes
anything from this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg use it, and only as the checker / the
reported CPU baseline.

The reference (HipKittens, ``/root/reference``) contains no MoE code at all: no
router, histogram, permutation, grouped GEMM, SiLU epilogue or combine.  Its
only FP8 GEMM semantics are the dequantise-then-fp32-matmul CPU loops of
``kernels/cdna4/gemm/mxfp8/MXFP8_4wave/4_wave.cu:466-478`` and the ``A @ B.T``
convention of
``kernels/cdna3/gemm/fp8fp32/mi300x/8192_256_256_64_32/data_logs/0613_003858_outputs/test_python.py:39-48``.
This package therefore restates those semantics for the dense GEMM and freezes
a written specification for everything the reference lacks.  Each function
cites what it follows; how each one is pinned (library routines, closed forms,
brute force) is listed in ``tests/test_oracle.py``.

Modules
-------
fp8     OCP e4m3fn decode/encode (RNE, saturating) and bf16 RNE, from the bit
        formats.
spec    quantisers, routing (top-k + softmax), expert offsets, permutation,
        dense/grouped GEMMs, SiLU*up, requantisation, combine, the full layer.
mx      MX (1x32 e8m0) quantiser, the reference's two-step scale packing,
        this path's one-step packing, and the MX dequantise-then-matmul GEMM.
brute   independent per-token brute-force restatement of the layer (no
        permutation, pure Python loops) used to pin ``spec`` on tiny shapes.
synth   seeded synthetic inputs for every configuration (numpy PCG64).
"""
