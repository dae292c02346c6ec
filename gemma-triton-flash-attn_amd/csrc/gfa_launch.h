// Internal launcher declarations (host side). Each returns the HIP status of the launch.
#pragma once
#include <hip/hip_runtime.h>
#include "gfa_params.h"

namespace gfa {

hipError_t launch_fwd(const FwdParams& p, int head_dim, int block_kv, int nwaves, bool bf16, bool cap, bool drop,
                      hipStream_t stream);
hipError_t launch_bwd_dq(const BwdDqParams& p, int head_dim, int block_kv, int split, bool bf16, bool cap, bool drop,
                         hipStream_t stream);
hipError_t launch_bwd_dkv(const BwdDkvParams& p, int head_dim, int block_q, int waves, int roles, bool bf16, bool cap,
                          bool drop, hipStream_t stream);
hipError_t launch_dkv_reduce(const BwdDkvParams& p, int head_dim, bool bf16, hipStream_t stream);
hipError_t launch_delta(const DeltaParams& p, bool bf16, hipStream_t stream);
hipError_t launch_bwd_dq_ds(const BwdDqDsParams& p, int head_dim, bool bf16, hipStream_t stream);

}  // namespace gfa
