/* Test infrastructure: dumps the reference's policy tree (src/model.h:9-3462)
 * as raw little-endian binary so tests can run the oracle's tree walk on the
 * very table the reference's model.so uses.  Built and run only where the
 * reference checkout is mounted; its output lives in oracle/_ref/ only.
 * Usage: policy_dump <out.bin>
 * Layout: int32 n_nodes, int32 n_cands, int32 root_fp16, int32 root_tf32,
 *         n_nodes * {8 x int32, 3 x float32}, n_cands * {2 x float32}. */
#include <stdio.h>
#include <stdint.h>
#include "model.h"

int main(int argc, char **argv)
{
    if (argc < 2) return 2;
    FILE *f = fopen(argv[1], "wb");
    if (!f) return 1;
    int32_t hdr[4] = {(int32_t)(sizeof tilespmm_shared_nodes / sizeof tilespmm_shared_nodes[0]),
                      (int32_t)(sizeof tilespmm_model_candidates / sizeof tilespmm_model_candidates[0]),
                      2512, 3420};
    fwrite(hdr, sizeof hdr, 1, f);
    for (int i = 0; i < hdr[0]; ++i) {
        const tilespmm_policy_node *n = &tilespmm_shared_nodes[i];
        int32_t iv[8] = {n->feature, n->left_feature, n->right_feature, n->child0,
                         n->child1, n->child2, n->child3, n->missing_left_mask};
        float fv[3] = {n->cut, n->left_cut, n->right_cut};
        fwrite(iv, sizeof iv, 1, f);
        fwrite(fv, sizeof fv, 1, f);
    }
    fwrite(tilespmm_model_candidates, sizeof tilespmm_model_candidates, 1, f);
    fclose(f);
    return 0;
}
