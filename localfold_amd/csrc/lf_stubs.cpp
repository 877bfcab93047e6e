// Entry points not yet implemented: they fail loudly with LF_ERR_UNSUPPORTED.
#include "lf_context.h"
#include "lf_ops.h"
extern "C" {
int lf_evoformer_block(lf_context*, const lf_evoformer_block_args*) { return lf::set_error(LF_ERR_UNSUPPORTED, "not built yet"); }
int lf_evoformer_stack(lf_context*, const lf_evoformer_block_args*, const lf_evoformer_weights*, int) { return lf::set_error(LF_ERR_UNSUPPORTED, "not built yet"); }
int lf_pairformer_block(lf_context*, const lf_pairformer_block_args*) { return lf::set_error(LF_ERR_UNSUPPORTED, "not built yet"); }
}
