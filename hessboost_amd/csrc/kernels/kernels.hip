// The gfx950 code object: every kernel of the backend in one translation unit.
#include "index.hip"
#include "gradients.hip"
#include "histogram.hip"
#include "partition.hip"
#include "split.hip"
#include "grow.hip"
#include "predict.hip"

// The abi.h checksum this code object was built with (checked by the host
// library at module load).
extern "C" __device__ const unsigned int hbr_abi_stamp = HBR_ABI_STAMP;
