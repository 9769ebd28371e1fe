/* gfx950 code object of the DiT hot path: every kernel the C-ABI runtime
 * loads by name through hipModuleGetFunction. */
#include "kernels/common.h"
#include "kernels/elementwise.h"
#include "kernels/gemm.h"
#include "kernels/gemm_q.h"
#include "kernels/attention.h"
#include "kernels/lora.h"
