// Single translation unit for the standalone code object (--genco): the
// reference-named extern "C" kernels of the GEMV, attention and glue sources,
// loadable with hipModuleLoad / hipModuleGetFunction.
#include "gemv.hip"
#include "attention.hip"
#include "glue.hip"
