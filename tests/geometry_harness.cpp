// CPU harness for the launch geometry (ace-kernels_amd/csrc/ace_geometry.hpp),
// the host arithmetic that picks each kernel's grid, block size and LDS.
// Built with g++ by tests/test_geometry.py and called through ctypes.
#include <cstdint>

#include "ace_geometry.hpp"

extern "C" {

// make_geometry of the fast forward (softmax, class labels; soft binning in
// the moments layout): block size, vector width, dynamic LDS of the forward
// and backward kernels, and blocks.  out: {nt, vec, lds_fwd, lds_bwd, nblk}.
void fast_geometry(long long B, long long C, long long N, int K, int soft, int include_background,
                   int max_nt, long long* out) {
  const ace::Geometry g = ace::make_geometry(B, C, N, K, soft != 0, include_background != 0, true, 0,
                                             0, soft != 0, true, max_nt);
  out[0] = g.nt;
  out[1] = g.var.vec;
  out[2] = (long long)g.lds_fwd;
  out[3] = (long long)g.lds_bwd;
  out[4] = g.nblk;
}

// Fraction bits of the generic soft kernels' fixed-point sums.
int soft_frac(long long voxels) { return ace::soft_frac(voxels); }

// The launch bound of the fast forward kernel that serves C channels.
int fast_bound(long long C, int soft) { return ace::fast_fwd_bound(ace::variant_for(C).cmax, soft != 0); }

}  // extern "C"
