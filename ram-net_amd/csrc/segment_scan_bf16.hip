// Segment scan kernels for bf16_t activations (one translation unit per dtype
// so the lane-layout instantiations compile in parallel).
#include "segment_scan.hpp"
#include "segment_scan_pair.hpp"

namespace ramnet {

hipError_t launch_scan_bf16(const SegmentJob &job, const ScanGeom &geo, int vec, int epp, int np, int nw, bool pre,
                          hipStream_t stream) {
    return scan_dispatch<bf16_t>(job, geo, vec, epp, np, nw, pre, stream);
}

hipError_t launch_scan_pair_bf16(const SegmentJob &job, const ScanGeom &geo, int vec, int epp, int nw,
                               hipStream_t stream) {
    return scan_pair_dispatch<bf16_t>(job, geo, vec, epp, nw, stream);
}

}  // namespace ramnet
