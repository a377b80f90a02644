"""CPU oracle for the rdv hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what the reference's kernels compute, each
function citing the reference file:line it follows.  It is the checker the
parity tests compare the HIP kernels against, and the CPU baseline bench.py
times beside them.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it; the product package (rdv_project_amd) never
does, and has no CPU fallback.

Modules:
  mlp        LinearFast / Linear / ReLU chains, the FREQ encoding, output heads
  winograd   F(2x2,3x3) convolution and the direct convolution it must equal
  render     camera rays, ray-box clipping, ray-marched transmittance,
             emission-absorption compositing
  train      MLP forward + backward with an MSE loss
  tensor_ops LinearTensorOp* / ReLUTensorOp
"""
