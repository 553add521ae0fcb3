// Host-side planning of split ranks (declared in common.h): how many of the longest causal
// chains of a prefill or backward grid run as two workgroups.
#include <math.h>

#include "common.h"

namespace mykfa {

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static int cached[kMaxDevices] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return 256;
    }
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cached[dev] = n;
    }
    return cached[dev];
}

int split_ranks(int gx, int seqs, int groups, int64_t rows, int blk, bool varlen, bool causal, int wgs_per_cu,
                size_t part_bytes) {
    if (!causal || gx < 8 || seqs <= 0 || groups <= 0 || blk <= 0 || part_bytes == 0) return 0;
    const double slots = (double)device_cu_count() * (wgs_per_cu > 0 ? wgs_per_cu : 1);
    const double g = gx;
    double share;
    if (!varlen) {
        share = groups * (double)seqs * g * (g + 1) / 2 / slots;
    } else {
        const double nb = (double)rows / blk;
        const double lb = groups * (g * (g + 1) / 2 + (nb > g ? nb - g : 0.0)) / slots;
        const double ub = groups * nb * (g + 1) / 2 / slots;
        share = sqrt(lb * ub);
    }
    int sr = gx - (int)ceil(share);
    if (sr > gx / 2) sr = gx / 2;
    if (sr <= 0) return 0;
    const size_t per_rank = (size_t)seqs * groups * 2 * part_bytes;
    const size_t fit = kSplitWorkspaceCap / per_rank;
    if ((size_t)sr > fit) sr = (int)fit;
    return sr;
}

}  // namespace mykfa
