// Single translation unit of libdsa_mli.so: the kernels share device
// functions and globals (the decode launch runs the top-k select; phase
// timestamps), which HIP resolves only within one unit without
// relocatable device code.
#include "topk.hip"
#include "decode_main.hip"
#include "scan_flat.hip"
#include "quant.hip"
#include "capi.hip"
#include "sol.hip"
