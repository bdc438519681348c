// Caller-side use of the C++ façade, written the way main.mm's cpu-bench
// and gpu-bench drive the reference (main.mm:478-509, 2704-2709).
#include <cstdio>
#include <cstring>

#include "mdnav.hpp"
#include "mdnav_host.h"

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: facade_example RAPTOR_BIN [envs] [rollouts] | --policy NAVPOL1_FILE\n");
        return 2;
    }
    if (std::strcmp(argv[1], "--policy") == 0 && argc > 2) {  // the deployed-policy loader, no GPU needed
        try {
            mdnav::NavigationPolicy policy;
            policy.load(argv[2]);
            std::printf("mode=%u observations=%u weights=%zu max_speed=%.2f source=%016llx\n",
                        policy.metadata.policy_mode, policy.metadata.observation_count, policy.weights.size(),
                        policy.metadata.max_speed_mps, (unsigned long long)policy.source_hash);
        } catch (const std::exception& e) {
            std::fprintf(stderr, "ERROR: %s\n", e.what());
            return 1;
        }
        return 0;
    }
    MdnRaptorWeights raptor;
    if (!mdn::load_raptor_file(argv[1], &raptor)) { std::fprintf(stderr, "RAPTOR load failed\n"); return 2; }
    MdnSimConfig cfg = mdn::default_config();
    cfg.n = argc > 2 ? uint32_t(std::atoi(argv[2])) : 128;
    cfg.family = 1; cfg.speed = 1; cfg.distance = 3;
    const uint32_t rollouts = argc > 3 ? uint32_t(std::atoi(argv[3])) : 2;
    try {
        mdnav::Trainer trainer(cfg, 32, raptor, mdn::crazyflie_params());
        // cpu_reference_benchmark checks the batched forward before training (main.mm:491)
        std::printf("validate_batched_forward=%d strict=%d\n", int(trainer.validate_batched_forward()),
                    int(trainer.validate_batched_forward(1e-9f)));
        const MdnMetrics m = trainer.run(rollouts);
        std::printf("envs=%u rollouts=%u wall_s=%.4f updates=%llu episodes=%llu ratio=%.4f\n", cfg.n, rollouts,
                    m.wall_seconds, (unsigned long long)m.updates, (unsigned long long)m.episodes, m.ratio);
        const mdnav::PPOTrainer::GradNormSummary g = trainer.ppo.grad_norm_summary();
        std::printf("grad_norm actor_mean=%.9g actor_max=%.9g actor_clip_frac=%.9g critic_mean=%.9g "
                    "critic_max=%.9g critic_clip_frac=%.9g\n",
                    g.actor_mean, g.actor_max, g.actor_clip_frac, g.critic_mean, g.critic_max, g.critic_clip_frac);
        trainer.sim.report("facade-train", 0);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ERROR: %s\n", e.what());
        return 1;
    }
    return 0;
}
