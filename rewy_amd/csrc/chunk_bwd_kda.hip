// fdr_chunk_bwd's KDA kernel (vector gate, scalar beta, K-first states, dense rows) in a
// translation unit of its own, so that build.py can give it its own machine scheduler (the
// kernel and its launcher are those of chunk_bwd.hip).
#define REWY_CHUNK_KDA_TU 1
#include "chunk_bwd.hip"
