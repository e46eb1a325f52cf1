"""CPU oracle for the FP8-blockwise fused-MoE layer.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
directory: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the reference the GPU
results are compared with (or the timed CPU baseline), never as the computation
that is shipped or measured.

It restates, in numpy, the CPU fallbacks of the reference plugin
(jinhuang12/vllm-neuron) for this path:

* router (topk -> activation -> scatter)   vllm_neuron/functional/moe/router.py:384-599
* blockwise mapping (align-by-expert)      vllm_neuron/functional/moe/moe_blockwise.py:91-157,325-498
* expert MLP, POST_SCALE accumulation      vllm_neuron/functional/moe/moe_cte.py:440-612
* fused decode block (norm/router/experts) vllm_neuron/functional/moe/moe_block_tkg.py:57-303
* scatter-add combine                      vllm_neuron/functional/moe/topk_reduce.py:144-159

and extends them with semantics the reference does not hold on any CPU path
(DeepSeek-style grouped sigmoid routing with a selection-only correction
bias; OCP e4m3fn 128x128 weight and 1x128 activation quantization), restated
from the public model definitions and pinned by closed forms, brute force and
library routines in ``tests/test_oracle_*.py``.

Parity status per function (what pins it):

* fp8.e4m3fn_encode/decode       all 256 codes and random/midpoint values vs torch.float8_e4m3fn
* fp8.quant_act_1x128/quant_w    amax element -> +-448, scale = amax/448, decode error bounds
* mathfn.exp_f32/sigmoid_f32     max ulp error vs float64 numpy (closed form)
* router.*                       brute-force sort / exhaustive group subsets on tiny inputs,
                                 invariants, torch.topk/softmax/sigmoid closed forms
* blockwise.*                    Python-loop brute force and invariants, docstring KATs
* moe.*                          float64 brute force on tiny shapes, dense == sparse form,
                                 linearity, permutation invariance
* moe.topk_reduce                docstring example of topk_reduce.py:70-82 (KAT)
* router.rms_norm_padded         constant rows (closed form), scale invariance at eps 0,
                                 equals rms_norm at hidden_actual = H, zero padding
* router.route_topk_scatter_act  same ids as a full sort; softmax weights equal the float64
                                 softmax of the selected logits; sigmoid rows 0 off the top-k
* moe.moe_block_tkg_fp8          NO_SCALE over all experts equals the dense all-expert form
                                 (moe_dense_reference, unit affinities); token permutation

The nkilib device kernels the reference calls (router_topk,
find_nonzero_indices, indexed_flatten, moe_cte, moe_block_tkg) are absent
from the reference snapshot; their internal accumulation order is parity
unpinned and the oracle follows the torch fallbacks instead.
"""
