// The gfx950 code object: every kernel of the backend in one translation unit.
#include "index.hip"
#include "gradients.hip"
#include "histogram.hip"
#include "partition.hip"
#include "split.hip"
#include "predict.hip"
