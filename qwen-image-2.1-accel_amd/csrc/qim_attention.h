// Host-side interface the attention entry points share (qim_attention.hip and
// the no-allocation entry point, qim_attention_noalloc.hip).
#pragma once

#include <stdint.h>

namespace qim {

// How one attention problem is run: workgroups [0, nfull) run whole work
// items, the ntail items after them run as nsplit chunks of kbc key blocks;
// the workspace holds the V^T tiles (vt_bytes), then the chunks' bf16 output
// rows (part_o_bytes) and fp32 (m, l) pairs (part_ml_bytes).
struct AttPlan {
    int64_t nfull, ntail, nsplit, kbc;
    int64_t vt_bytes, part_o_bytes, part_ml_bytes;
    int64_t total() const { return vt_bytes + part_o_bytes + part_ml_bytes; }
};

// The plan of a (B, S, T, H) problem on the current device.
AttPlan att_plan(int64_t B, int64_t S, int64_t T, int64_t H);

// Checks the arguments and launches the attention kernels (see qim.h,
// qim_attention / qim_attention_mxfp8); `who` names the entry point in errors.
int attention_run(const char *who, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v,
                  int64_t ldv, void *o, int64_t ldo, void *qcodes, void *qscales, int tiled, void *workspace,
                  int64_t workspace_bytes, int64_t B, int64_t S, int64_t T, int64_t H, int64_t D, float scale,
                  void *stream);

}  // namespace qim
