// A 60-comparator, depth-10 sorting network for 16 inputs (the optimal size
// known for n = 16).  Plain C++ so the host test suite can check it
// exhaustively with the 0-1 principle (tests/test_sortnet.py).
#pragma once

namespace glsdm {

constexpr int SORTNET16_SIZE = 60;
constexpr unsigned char SORTNET16[SORTNET16_SIZE][2] = {
    {0, 13}, {1, 12}, {2, 15}, {3, 14}, {4, 8}, {5, 6}, {7, 11}, {9, 10},
    {0, 5}, {1, 7}, {2, 9}, {3, 4}, {6, 13}, {8, 14}, {10, 15}, {11, 12},
    {0, 1}, {2, 3}, {4, 5}, {6, 8}, {7, 9}, {10, 11}, {12, 13}, {14, 15},
    {0, 2}, {1, 3}, {4, 10}, {5, 11}, {6, 7}, {8, 9}, {12, 14}, {13, 15},
    {1, 2}, {3, 12}, {4, 6}, {5, 7}, {8, 10}, {9, 11}, {13, 14},
    {1, 4}, {2, 6}, {5, 8}, {7, 10}, {9, 13}, {11, 14},
    {2, 4}, {3, 6}, {9, 12}, {11, 13},
    {3, 5}, {6, 8}, {7, 9}, {10, 12},
    {3, 4}, {5, 6}, {7, 8}, {9, 10}, {11, 12},
    {6, 7}, {8, 9},
};

}  // namespace glsdm
