// Test library: the one-pass scan's bounded wait giving up, forced from the host
// with every kernel exiting normally.
//
// probe_scan_unit_timeout scans n elements (two units: 16384 < n <= 32768) with
// a workspace whose unit counter the host starts at 1 and a grid of one
// workgroup. That workgroup takes unit 1, whose prefix needs unit 0's total;
// unit 0 never runs, so its slot is never published and the wait gives up
// after `spin_limit` polls. The unit must then count the timeout in workspace
// word 1 and write NaN to all of its outputs, for the prefix sum and for the
// prefix maximum (whose fmaxf would otherwise drop a NaN carry). Unit 0's
// outputs are left untouched.
#include <opworks>

#include <cstdint>

namespace {

__global__ void start_counter_kernel(uint32_t *ws, uint32_t first_unit) { ws[0] = first_unit; }

template <typename Op> void run(const float *in, float *out, uint32_t *ws, int n, int spin_limit, hipStream_t s) {
    using namespace opworks::detail;
    const ScanLayout lay = scan_pair_layout(n);
    const int64_t quads = (lay.words() + 3) / 4;
    opworks::launch_async(s, scan_clear_kernel, static_cast<int>(blocks_for64(quads, 256)), 256,
                          reinterpret_cast<uint4 *>(ws), quads);
    opworks::launch_async(s, start_counter_kernel, 1, 1, ws, 1u);
    opworks::launch_async(s, scan_pair_kernel<Op, true, true, true>, 1, kScanThreads, in, out, ws, lay,
                          static_cast<int64_t>(n), spin_limit);
}

} // namespace

extern "C" {

// Workspace words the probe needs for n elements (the scan's own layout).
int probe_scan_workspace_words(int n) {
    return static_cast<int>(opworks::detail::scan_pair_layout(n).words());
}

// Returns 0 once the kernels are enqueued and the stream drained; -1 for an n that is not two units
// or a spin limit outside [0, 2^18].
int probe_scan_unit_timeout(const float *in, float *out, uint32_t *ws, int n, int maximum, int spin_limit,
                            void *stream) {
    using namespace opworks::detail;
    if (n <= kScanPair || n > 2 * kScanPair || spin_limit < 0 || spin_limit > kScanSpinLimit)
        return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (maximum)
        run<ScanMaxOp>(in, out, ws, n, spin_limit, s);
    else
        run<ScanSumOp>(in, out, ws, n, spin_limit, s);
    OPWORKS_HIP_CHECK(hipStreamSynchronize(s));
    return 0;
}

} // extern "C"
