// CPU check of the attention kernels' work-item order (attn_item in
// common.cuh): for every grid of G items (nb blocks per head) and every slot
// count, workgroup L -> item attn_item(L, G, nb, slots) must be a
// permutation of 0 .. G - 1, or some (b, h, block) would be computed twice
// and another never. Built for the host only by tests/test_host.py; prints
// the number of grids checked, exits 1 on the first failure.
#include <cstdio>
#include <vector>

#include "../memory_efficient_attn_layer_amd/csrc/common.cuh"

int main() {
  long grids = 0;
  const int nbs[] = {1, 2, 3, 7, 16, 32, 33, 64, 256};
  for (int nb : nbs)
    for (int heads = 1; heads <= 600; heads += (heads < 40 ? 1 : 37)) {
      const int G = heads * nb;
      for (int slots = 1; slots <= 4; ++slots) {
        std::vector<int> seen(G, 0);
        for (int L = 0; L < G; ++L) {
          const int it = mea::attn_item(L, G, nb, slots);
          if (it < 0 || it >= G || seen[it]++) {
            std::printf("FAIL G=%d nb=%d slots=%d L=%d item=%d\n", G, nb, slots, L, it);
            return 1;
          }
        }
        ++grids;
      }
    }
  std::printf("ok %ld grids\n", grids);
  return 0;
}
