"""CPU oracle for the fused 2:4-sparse Conv+BN+LIF path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or as the timed CPU baseline).  The product
(sparsesnn_amd) never imports it and has no CPU fallback.

Modules:
  reference_path — restatement of the SparseSNN PyTorch path (models/neurons.py,
                   models/layers.py, sparse/pruning.py, sparse/utils.py,
                   sengine/optimizer.py BN fold / 2:4 check), run on torch CPU fp32.
  packing        — numpy restatement of the spike-bit format and of the 2:4 / dense
                   weight blobs consumed by the gfx950 kernels (net-new formats; pinned
                   by round trips and known-answer placements in tests/test_oracle.py).

Pinning status (what checks each function; see tests/test_oracle.py):
  prune_n_m / prune_conv_2_4   brute-force per-group top-2 on small tensors, invariants
  verify_n_m / validate_2_4    hand-built pass/fail cases
  fold_batchnorm               closed form in float64 vs eval BatchNorm
  conv_bn_seq                  float64 brute-force direct convolution (stride, pad, dilation)
  multistep_lif / multistep_if closed forms (no-spike geometric series, constant-drive
                               spike trains), soft/hard reset hand traces
  fused_layer                  composition of the above + committed cfg0 golden fixture
  packing.*                    pack/unpack and compress/decompress round trips,
                               known-answer slot placement, plane reconstruction bound
"""
