// Caller-side use of the navigation_training façade (include/mdnav.hpp),
// written the way main.mm's task commands drive the reference
// (navigation_training::evaluate / train).
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "mdnav.hpp"
#include "mdnav_host.h"

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr,
                     "usage: training_example --task-eval RAPTOR_BIN CHECKPOINT STAGE FAMILY AMPLITUDE SEED CSV\n"
                     "       training_example --task-train RAPTOR_BIN CHECKPOINT WARMSTART ROLLOUTS STAGE FAMILY "
                     "AMPLITUDE SEED\n");
        return 2;
    }
    mdnav::Context ctx;
    if (!mdn::load_raptor_file(argv[2], &ctx.raptor)) {
        std::fprintf(stderr, "RAPTOR load failed\n");
        return 2;
    }
    ctx.physics = mdn::crazyflie_params();
    try {
        if (std::strcmp(argv[1], "--task-eval") == 0 && argc == 9) {
            MdnCheckpointHeader h{};
            mdnav::require(mdn_checkpoint_read_params(argv[3], &h, nullptr, 0, nullptr, 0));
            std::vector<float> actor(h.actor_count);
            mdnav::require(mdn_checkpoint_read_params(argv[3], &h, actor.data(), actor.size(), nullptr, 0));
            const auto score = mdnav::navigation_training::evaluate(
                ctx, actor.data(), uint32_t(std::atoi(argv[4])), uint32_t(std::atoi(argv[5])),
                float(std::atof(argv[6])), uint32_t(std::strtoul(argv[7], nullptr, 10)), argv[8]);
            std::printf("score success=%.6f collision=%.6f timeout=%.6f arrival=%.6f\n", score.success,
                        score.collision, score.timeout, score.successful_time_s);
            return 0;
        }
        if (std::strcmp(argv[1], "--task-train") == 0 && argc == 10) {
            mdnav::navigation_training::train(ctx, uint32_t(std::atoi(argv[5])), argv[3], argv[4],
                                              uint32_t(std::atoi(argv[6])), uint32_t(std::atoi(argv[7])),
                                              float(std::atof(argv[8])), uint32_t(std::strtoul(argv[9], nullptr, 10)));
            std::printf("trained\n");
            return 0;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ERROR: %s\n", e.what());
        return 1;
    }
    std::fprintf(stderr, "bad arguments\n");
    return 2;
}
