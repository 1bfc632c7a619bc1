/* Umbrella header of the CBSAttn module: the C ABI of libbsattn.so. */
#include "../../../include/bsattn.h"
