// policy_model.h -- (gamma, delta) policy table for MI355X.
//
// Node layout and walk semantics are those of the reference's exported
// decision tree (tilespmm_policy_node, src/model.h:9-13; walk
// src/model.h:3463-3491) so that a retrained table drops into the same
// tilespmm_predict_* C ABI.  Action a selects candidate a of the list built
// by policy_candidates().
//
// PROVISIONAL TABLE: a single leaf per precision until the exhaustive MI355X
// tuning sweep (every candidate x the benchmark matrices) has been run and a
// tree fitted to it.  The leaf is the candidate that the tuning sweep is
// expected to start from: gamma = 2.0, delta = 1.5.
#pragma once

struct tsp_policy_node {
    int feature, left_feature, right_feature;
    int child0, child1, child2, child3, missing_left_mask;
    float cut, left_cut, right_cut;
};

// One placeholder node (never reached: both roots are leaves).
static const tsp_policy_node tsp_policy_nodes[] = {
    {4, -1, -1, -1, -1, -1, -1, 0, 0.0f, 0.0f, 0.0f},
};

// A root < 0 is a leaf holding action -1 - root.
static const int tsp_policy_root_fp16 = -1 - 24;   // candidate 24: (2.0, 1.5)
static const int tsp_policy_root_tf32 = -1 - 24;
