"""CPU oracle for the Evoformer / Pairformer pair-stack path.

TEST INFRASTRUCTURE ONLY.  Nothing in `localfold_amd/` imports, links or runs this
package: only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` use it, and only as the checker (or the timed CPU baseline), never as the
thing measured or shipped.

It restates, in numpy, the reference's CPU path for the hot path:

* `webgpu/kernels/triangle/cpu-reference.js`  - AF2 triangle multiplication
* `cpu/af3/trunk/pairformer.js`               - AF3 layer norm, linear, transition,
                                                triangle multiplication, grid and single
                                                attention, pairformer block
* `cpu/af3/trunk/msa.js`                      - AF3 outer-product-mean
* AF2-only semantics the reference states only as WGSL (`webgpu/kernels/attention.js`,
  `transition.js`, `outer-product-mean.js`, `webgpu/af2/evoformer/block.js`)
* the weight codecs of `shared/weights/dtype.js` and the quantisers of
  `tools/quantize_af3.py` / `tools/quantize_model.py`
* the deterministic generator of `webgpu/testing/deterministic-input.js`

Arithmetic follows the reference's JS: every intermediate is computed in float64 (JS
numbers) and stored as float32 (`Float32Array`) at the same points the reference stores
it.  Each function cites the reference file:line it follows.

Pinning status (what checks each function, in tests/test_oracle.py and, for the AF3
functions, tests/test_oracle_af3.py):

* tri_mult_af2 outgoing   - the four committed fixtures (OpenFold + three AlphaFold captures)
* tri_mult_af2 incoming   - transpose identity against outgoing on the same fixtures,
                            plus a brute-force einsum on tiny inputs
* tri_mult_af3            - reduction to tri_mult_af2 with interleaved weights / no biases
                            (closed form), and the transposed identity
* layer_norm / linear     - closed forms (row independence, transposed weights, scale)
* attention (all modes)   - brute-force per-element softmax loops on tiny inputs;
                            invariants: one unmasked key -> that value row; transpose
                            identity; zero bias -> plain attention
* outer_product_mean_af2  - S=1 closed form; the count identity at S=5 with ragged
                            masks (constant LN output, so the sum over sequences is the
                            coverage count times one outer product); a per-element loop
                            at S=4
* outer_product_mean_af3  - the reference's hand-computed cases (`test/af3-msa.test.js:40-107`:
                            sum before divide, per-pair coverage, uncovered pair = 0,
                            asymmetry) plus channel order and bias-before-divide
* global_column_attention_af2 - per-element loops of the four kernels of
                            `webgpu/af2/evoformer/block.js:101-400` (64-lane online softmax);
                            a two-sequence closed form that fixes 1/sqrt(d), the masked mean
                            and the -1e9; permutation and masked-sequence invariants
* msa_pair_weighted_averaging_af3 - a per-element loop of `msaAttention` on an asymmetric
                            pair (the [h][i][j] orientation); one-token, zero-logit, deleted-
                            token and all-masked closed forms
* single_attention_af3    - per-element loops of `singleAttention` on tiny inputs; a
                            two-token closed form that fixes the 1/sqrt(d) scale, the q bias
                            and the pair logit; masked-key and one-unmasked-key invariants
* grid_self_attention_af3 - per-element loops of `gridSelfAttention` (starting, ending,
                            ending with the swapped bias) on an asymmetric mask; a closed
                            form that fixes the scale and the key mask
* transitions             - closed forms (ReLU split, SwiGLU blocked split, swish(1))
* codecs                  - the reference's own int5 boundary cases
                            (`test/int5-tensor.test.js`), quantise->decode round trips
* generator               - integer restatement (counter form), checked against a direct
                            sequential loop
* pairformer block order  - the single track reads the pair after all five pair updates
                            (reading it before the pair transition fails the check)
* evoformer block order   - composition of the pinned ops (parity of the
                            composition itself is pinned only by that construction:
                            the reference's block fixtures are absent from its checkout)
"""
