// Host-side exports of the LDS row layouts (race_layout.h) for the layout
// tests.  Built with g++ -D__host__= -D__device__= (pure integer functions).
#include "../../race_attention_amd/csrc/race_layout.h"

extern "C" int race_sw_pitch(int n) { return race::layout::sw_pitch(n); }
extern "C" int race_sw_elem(int n, int r, int e) { return race::layout::sw_elem(n, r, e); }
extern "C" int race_pi_pos(int k) { return race::layout::pi_pos(k); }
