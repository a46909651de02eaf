// random.h -- the process-wide generator of parameter initialisers
// (include/inferno/util/random.h, src/inferno/util/random.cpp of the reference).
// Same interface over std::mt19937; uniform draws as the reference's, plus
// normal draws (no reference counterpart) for N(0, sigma^2) initialisation.
#pragma once
#include <cstddef>
#include <vector>

namespace Inferno {

class RandomGenerator {
public:
    static void initialize();                         // non-deterministic seed
    static void initializeWithSeed(unsigned int seed);
    static std::vector<float> generateRandomFloatVector(size_t size, float minValue = 0.0f, float maxValue = 1.0f);
    static std::vector<double> generateRandomDoubleVector(size_t size, double minValue = 0.0, double maxValue = 1.0);
    static std::vector<int> generateRandomIntVector(size_t size, int minValue = -1, int maxValue = 1);
    static float generateRandomFloat(float minValue = 0.0f, float maxValue = 1.0f);
    static double generateRandomDouble(double minValue = 0.0, double maxValue = 1.0);
    static int generateRandomInt(int minValue = -1, int maxValue = 1);
    static std::vector<float> generateNormalFloatVector(size_t size, float mean, float stddev);
};

}  // namespace Inferno
