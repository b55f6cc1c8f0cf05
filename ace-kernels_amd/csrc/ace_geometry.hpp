// Launch geometry and device-memory layout shared by the host dispatch and the
// kernels.  Host-only arithmetic; no HIP calls.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace ace {

constexpr int kThreads = 256;           // threads per block (4 wave64); the epilogue's width
constexpr int kFastThreads = 1024;      // threads per block of the fast forward kernels (16 wave64)
constexpr int kFrac = 30;               // fixed-point fraction bits of the sums
constexpr int kMaxChannels = 64;        // largest C with a built kernel
constexpr size_t kMaxHistLds = 32 * 1024;  // default LDS budget of the histogram copies
constexpr int kMaxCopyCount = 2047;        // hard: voxels one copy may count (11-bit field)
constexpr int kMaxMomCopyCount = 4095;     // soft moments: the same (12-bit field)
constexpr int kCtrStride = 64;             // ints between ticket counters (one 256-byte line each)
constexpr int kGroupTiles = 16;            // blocks per ticket group
constexpr int kSingleTicketTiles = 256;    // up to this many blocks per batch index: one ticket level
constexpr int kRepTiles = 256;             // blocks per replica of the final sums
constexpr int kRepTilesFast = 64;          // the same for the fast forward's 1024-thread blocks
constexpr int kMaxReps = 4;                // replicas of the final sums per batch index
constexpr size_t kMaxFastHistLds = 150 * 1024;  // LDS budget of the histogram copies, 1024-thread blocks
constexpr int kFastCopies = 16;            // histogram copies of a 1024-thread block

// Channel variants with a compiled kernel: the kernel keeps C logits of VEC
// voxels in registers.  EXACT variants fix C at compile time; the others
// handle any C up to CMAX with uniform guards.  C = 16 takes one voxel per
// lane and step: its forward then holds 107 VGPRs instead of 184 and its
// backward 81 instead of 128, and on MI355X cfg 4's step went from 104 to
// 97.6 us (forward 47.2 -> 43.9 us).
struct Variant {
  int cmax;
  bool exact;
  int vec;  // voxels per thread and step
};

inline Variant variant_for(int64_t C) {
  if (C == 1) return {1, true, 4};
  if (C == 2) return {2, true, 4};
  if (C == 3) return {3, true, 4};
  if (C == 4) return {4, true, 4};
  if (C <= 8) return {8, false, 4};
  if (C == 16) return {16, true, 1};
  if (C <= 16) return {16, false, 4};
  if (C <= 32) return {32, false, 1};
  return {64, false, 1};
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Bytes of one histogram copy for a (C' * K)-bin block histogram.
//   hard: u64 packed (count | label count | sum p), plus an i64 sum of the
//         targets when they are per-channel values rather than labels
//   soft: three i64 fixed-point sums W, P, G
//   soft moments (softmax + labels): per half-bin (2K per channel) the packed
//         word (count | label count | sum u), sum u^2 and sum u over the
//         labelled voxels, u the offset of the quantised p from the
//         half-bin's base (moment_scale)
constexpr size_t hist_bytes_per_copy(int ck, bool soft, bool labels, bool moments = false) {
  return moments ? (size_t)ck * 48 : (soft ? (size_t)ck * 24 : (size_t)ck * (labels ? 8 : 16));
}

// Final sums per batch index and replica: 3 x C'K (W, P, G per bin); 2 x C'K
// for hard binning with class labels (W << 32 | G packed in one word, then
// P); for soft moments 5 x 2C'K (count, label count, sum u, sum u^2 >>
// shift, sum u over the labelled voxels per half-bin).
constexpr int fin_values(int ck, bool moments, bool packed = false) {
  return moments ? 10 * ck : (packed ? 2 * ck : 3 * ck);
}

// LDS layout of an epilogue over nb batch indices (byte offsets from the
// histogram region): d, W, G (float) and an empty flag per bin, the per-class
// errors, and for soft moments six float64 contributions per half-bin.
struct EpiLayout {
  size_t sf, terms, bytes;
};
constexpr size_t align16(size_t v) { return (v + 15) / 16 * 16; }
constexpr EpiLayout epi_layout(int ck, int cl, int nb, bool moments) {
  return EpiLayout{align16((size_t)13 * ck * nb),
                   align16(align16((size_t)13 * ck * nb) + (size_t)4 * cl * nb),
                   align16(align16((size_t)13 * ck * nb) + (size_t)4 * cl * nb) +
                       (moments ? (size_t)96 * ck * nb : 0)};
}
constexpr int kMaxEpiRows = 16;  // C' up to which a single batch index's epilogue sums the loss

// A problem streams when its logits, targets and gradient exceed
// kStreamBytes, 7/8 of MI355X's 256 MB last-level cache: the backward then
// writes the gradient with nontemporal stores, so that the gradient does not
// displace the logits that the forward left in that cache and the backward
// reads.  Below it the gradient's lines are written back from the cache
// after the kernel.  Separately, the hard forward reads the class labels
// with nontemporal loads at every size (the hard backward does not read
// them).  On MI355X, eager fwd+bwd step: cfg 4 (285 MB) -6 us with the
// streaming stores; cfg 2 (168 MB) -1.2 to -2.5 us with the label loads,
// +0.5 us with streaming stores.  Nontemporal logit loads in the forward
// too made cfg 4's step 10 us slower instead.
constexpr size_t kStreamBytes = (size_t)224 << 20;
inline bool stream_problem(size_t x_bytes, size_t target_bytes) {
  return 2 * x_bytes + target_bytes > kStreamBytes;
}

// Fraction bits of the generic soft kernels' fixed-point sums of weights,
// weight * p and weight * y (each term below 2): 40, or fewer for a batch
// index of more than 2^19 voxels, so that a bin's sum (at most N terms that
// add to at most N) stays below 2^61.  With 30 bits a small weight times p
// lost bits (exact only from 2^-7), and the soft gradient amplifies d's
// error by 2K / W in bins of a few voxels; with 40 the terms are exact from
// 2^-17.
inline int soft_frac(int64_t voxels) {
  int bits = 0;
  while (bits < 62 && (1ll << bits) <= voxels) ++bits;  // bit length of N
  const int f = 60 - bits;
  return f < 40 ? (f < 1 ? 1 : f) : 40;
}

// Channel counts served by the fast (softmax + class-index labels) kernels.
inline bool fast_channels(int64_t C) { return C == 2 || C == 3 || C == 4 || C == 16; }

// Launch bound of the fast forward kernel for C channels (its compile-time
// channel variant): kFastThreads for hard binning with C <= 4, kThreads
// otherwise (16 channels with two tiles in flight need more than the 128
// VGPRs of 16 waves per CU; soft moments run in 256-thread blocks).  The
// launchers refuse a block size above it, and make_geometry never picks one
// (tests/test_geometry.py checks every configuration the fast kernels serve).
constexpr int fast_fwd_bound(int C, bool soft) { return (C <= 4 && !soft) ? kFastThreads : kThreads; }

struct Geometry {
  Variant var;
  int nt;              // threads per forward block (kThreads, or kFastThreads for the fast kernels)
  bool fast;           // the forward runs a fast (softmax + class labels) kernel
  bool packed;         // hard binning with labels: W and G share one final-sum word
  int C, CL, off, K, ck;
  int64_t B, N;
  int steps;           // vector steps per block
  int64_t tile_vox;    // voxels per block (one batch index)
  int64_t tiles;       // blocks per batch index
  int64_t nblk;        // total blocks
  int64_t gs;          // blocks per ticket group
  int64_t gpb;         // groups per batch index
  int reps;            // replicas of each batch index's final sums
  int copies;          // histogram copies (lane % copies)
  int lchunk;          // log2 of the copies one lane adds in the block sums
  bool moments;        // soft binning through per-half-bin moments
  bool epi_all;        // one block runs the epilogue of every batch index
  size_t tab_floats;   // padded bucket table (n + 2) + centre table (2K + 2)
  size_t lds_fwd;      // dynamic LDS of the forward kernel
  size_t lds_bwd;      // dynamic LDS of the backward kernel
  size_t off_part;     // byte offset of the per-batch loss partial words
  size_t off_fin;      // byte offset of the final sums in the workspace
  size_t ws_bytes;     // workspace bytes; all of it starts zero and is left zero
};

// Blocks per batch index: aim for ~4 blocks of 256 threads per CU on a
// 256-CU part (the generic kernels), or one block of 1024 threads per CU (the
// fast forward kernels: softmax with class labels, `fast`), keeping every
// block's tile a whole number of vector steps.
// moments: the soft fast path (softmax + labels, fast_channels(C)) that bins
// per-half-bin moments instead of per-voxel weights.
inline Geometry make_geometry(int64_t B, int64_t C, int64_t N, int K,
                              bool soft, bool include_background, bool labels,
                              int steps_override = 0, int copies_override = 0,
                              bool moments = false, bool fast = false,
                              int max_nt = kFastThreads, bool backward = false) {
  Geometry g{};
  g.moments = moments;
  g.var = variant_for(C);
  // the fast hard forward at C = 4 takes two voxels per lane and step (61
  // VGPRs instead of 100): on MI355X cfg 2's forward 26.7 vs 27.8 us; the
  // soft and backward kernels measured slower that way and keep four
  if (fast && !soft && C == 4) g.var.vec = 2;
  // the generic kernels for 5-16 channels take one voxel per lane: at four,
  // soft held 283 VGPRs at 8 channels and spilled at 16, hard 209 and 392
  // (one or two waves per SIMD); the launchers instantiate them so.  The
  // hard backward for 5-8 channels takes two (MI355X, B = 2, C = 5, 128^3:
  // 58.3 us against 75.7 at one and 73.6 at four; every other generic kernel
  // measured fastest at one)
  if (!g.var.exact) g.var.vec = (backward && !soft && g.var.cmax == 8) ? 2 : 1;
  g.C = (int)C;
  g.off = (!include_background && C > 1) ? 1 : 0;
  g.CL = (int)C - g.off;
  g.K = K;
  g.ck = g.CL * K;
  g.B = B;
  g.N = N;
  g.packed = !soft && labels;
  const size_t per_copy = hist_bytes_per_copy(g.ck, soft, labels, moments);
  const bool counted = !soft || moments;  // copies count voxels in 11-bit fields
  // fast forward: 1024-thread blocks (one per CU) with up to kFastCopies
  // copies, as many as the LDS holds; each copy counts at most kMaxCopyCount
  // voxels (nt / copies lanes x steps x vec).  When even one vector step per
  // lane would overflow a copy, the fast kernel runs with 256-thread blocks.
  int fast_copies = 0, fast_steps_max = 0;
  if (fast) {
    int c = copies_override > 0 ? copies_override : kFastCopies;
    while (c > 1 && per_copy * c > kMaxFastHistLds) c /= 2;
    fast_copies = c;
    fast_steps_max = (int)((int64_t)kMaxCopyCount / ((int64_t)(kFastThreads / c) * g.var.vec));
  }
  g.fast = fast;
  // 1024 threads for hard binning with C <= 4 only: the 16-channel kernel's
  // registers allow 256, and soft moments measured slower in 1024-thread
  // blocks, whose 48 C'K-byte copies leave fewer copies per lane (MI355X,
  // cfg 3: 34.9 vs 34.5 us; cfg 5, 50 bins: 70.8 vs 51.2 us)
  g.nt = (fast && !soft && C <= 4 && fast_steps_max >= 1 && max_nt >= kFastThreads) ? kFastThreads
                                                                                      : kThreads;
  int copies;
  if (g.nt == kFastThreads) {
    copies = fast_copies;
  } else {
    // histogram copies (lane % copies), within the LDS budget: at most 8 for
    // hard binning and soft moments -- more copies cut LDS address conflicts
    // but lengthen the block sums, and on MI355X 8 measured fastest for hard
    // (cfg 2: 8 ~ 16 < 32 copies); soft moments fill the LDS budget at 8 --
    // and up to 32 for the generic soft sums
    copies = copies_override > 0 ? copies_override : ((soft && !moments) ? 32 : 8);
    while (copies > 1 && per_copy * copies > (copies_override > 0 ? 160 * 1024 : kMaxHistLds))
      copies /= 2;
  }
  g.copies = copies;
  const int64_t step_vox = (int64_t)g.nt * g.var.vec;
  int steps = steps_override;
  if (steps <= 0) {
    const int64_t total = B * (N > 0 ? N : 1);
    // generic kernels: ~4 blocks per CU; half that above 8 channels, whose
    // kernels hold ~120 VGPRs (4 waves per SIMD: 1024 blocks would just fill
    // the chip, and on MI355X ~10% of them started a round late) and issue
    // C x K x 3 final-sum atomics per block (cfg 4, C = 16: 52 us at 512
    // blocks vs 57 us at 1024).  Fast kernels: one 1024-thread block per CU.
    const int64_t target_blocks = g.nt == kFastThreads ? 256 : (C > 8 ? 512 : 1024);
    steps = (int)cdiv(total, step_vox * target_blocks);
    if (steps < 1) steps = 1;
    if (steps > 64) steps = 64;
  }
  const int64_t copy_cap = moments ? kMaxMomCopyCount : kMaxCopyCount;
  if (counted) {
    // every copy counts at most copy_cap voxels of a tile
    const int64_t max_steps = copy_cap * copies / step_vox;
    if (steps > max_steps) steps = (int)(max_steps > 0 ? max_steps : 1);
  }
  g.steps = steps;
  // block sums: a lane adds the packed words of as many copies as keep the
  // count fields within kMaxCopyCount before decoding them (a copy counts at
  // most nt / copies lanes x steps x vec voxels)
  const int64_t copy_vox = (int64_t)(g.nt / copies) * steps * g.var.vec;
  int chunk = copies;
  while (chunk > 1 && (!soft || moments) && chunk * copy_vox > copy_cap) chunk /= 2;
  int lchunk = 0;
  while ((1 << lchunk) < chunk) ++lchunk;
  g.lchunk = lchunk;
  g.tile_vox = step_vox * steps;
  g.tiles = N > 0 ? cdiv(N, g.tile_vox) : 1;
  g.nblk = B * g.tiles;
  // tickets: one counter per batch index when it has at most
  // kSingleTicketTiles blocks (one device-scope round trip fewer at the end),
  // else groups of kGroupTiles blocks, then the groups of a batch index; final
  // sums replicated so that ~kRepTiles blocks share a replica
  g.gs = g.tiles <= kSingleTicketTiles ? g.tiles : kGroupTiles;
  g.gpb = cdiv(g.tiles, g.gs);
  int64_t reps = cdiv(g.tiles, g.nt == kFastThreads ? kRepTilesFast : kRepTiles);
  g.reps = (int)(reps > kMaxReps ? kMaxReps : reps);
  const int n = soft ? 2 * K : K;
  g.tab_floats = align_up((size_t)(n + 2) + (soft ? (size_t)(2 * K + 2) : 0), 4);
  // the epilogue block reuses the histogram region (epi_layout).  With one
  // batch index its epilogue block also sums the loss (no loss ticket); with
  // more, batch epilogues run in parallel blocks (one block doing several
  // measured slower on MI355X), then the last one sums the loss.
  const size_t hist = align_up(per_copy * copies, 16);
  g.epi_all = B == 1 && g.CL <= kMaxEpiRows;
  const size_t epi = epi_layout(g.ck, g.CL, 1, moments).bytes;
  const size_t region = hist > epi ? hist : epi;
  g.lds_fwd = g.tab_floats * 4 + region;
  // backward: tables + coef (+ d's two parts) + g, then for soft moments
  // nine values per half-bin from a 16-byte boundary (bwd_fast_body)
  g.lds_bwd = (align_up(g.tab_floats + (size_t)g.ck * (soft ? 3 : 1) + (size_t)g.CL, 4) +
               (moments ? 18 * (size_t)g.ck : 0)) * 4;
  // workspace: ticket counters (groups, batch indices, loss), one loss
  // partial word per batch index and the final sums; it must start zero and
  // every call leaves it zero
  const int64_t counters = B * g.gpb + B + 1;
  g.off_part = align_up((size_t)counters * kCtrStride * sizeof(int), 256);
  g.off_fin = align_up(g.off_part + (size_t)B * sizeof(unsigned long long), 256);
  const size_t fin_bytes = (size_t)B * g.reps * fin_values(g.ck, moments, g.packed) * sizeof(unsigned long long);
  g.ws_bytes = align_up(g.off_fin + fin_bytes, 256);
  return g;
}

}  // namespace ace
