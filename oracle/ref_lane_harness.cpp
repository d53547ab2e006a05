// Exports the reference's own trellis lane-window code (engine/exl3/kernels/lane_window.h,
// compiled from where it lies under the reference root) so the tests can check this
// repository's CPU oracle against it.  Test infrastructure only; built into oracle/_ref/.
#include "engine/exl3/kernels/lane_window.h"

template <int K>
static void Run(int t, const uint32_t* words, uint32_t* st, int* d0, int* shift) {
  const crucible::LaneWindow<K> win(t);
  constexpr int T = crucible::TileDwords(K);
  crucible::LaneStates<K>(words[win.d0], words[(win.d0 + 1) % T], words[(win.d0 + 2) % T], win.shift, st);
  *d0 = win.d0;
  *shift = win.shift;
}

// k_code: the reference's width code (1..8, or 15/25/35 for K = 1.5/2.5/3.5).
// words: one tile's dwords; t: lane 0..31; st: 8 states (low 16 bits valid).
extern "C" int ref_lane_states(int k_code, int t, const uint32_t* words, uint32_t* st, int* d0, int* shift) {
  switch (k_code) {
    case 1: Run<1>(t, words, st, d0, shift); return 0;
    case 2: Run<2>(t, words, st, d0, shift); return 0;
    case 3: Run<3>(t, words, st, d0, shift); return 0;
    case 4: Run<4>(t, words, st, d0, shift); return 0;
    case 5: Run<5>(t, words, st, d0, shift); return 0;
    case 6: Run<6>(t, words, st, d0, shift); return 0;
    case 7: Run<7>(t, words, st, d0, shift); return 0;
    case 8: Run<8>(t, words, st, d0, shift); return 0;
    case 15: Run<15>(t, words, st, d0, shift); return 0;
    case 25: Run<25>(t, words, st, d0, shift); return 0;
    case 35: Run<35>(t, words, st, d0, shift); return 0;
    default: return -1;
  }
}
