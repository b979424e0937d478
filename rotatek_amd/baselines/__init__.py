"""ThinK and SparK channel-pruning baselines on the HIP device
(drop-in for rotatek/baselines/ and for the recovery step of the model
adapters, llama_visionzip.py:216-233).

* ``think.think_score_and_compact``   think.py:15-58
* ``spark.per_token_channel_prune``   spark.py:15-60
* ``recover.recover_think`` / ``recover.recover_spark``
                                      full-width visual Keys for the dense
                                      decode (optionally with the prompt and
                                      text rows in the same pass)
* ``recover.selection_rotation``      one-hot R from a ThinK keep mask, so
                                      the RotateK decode kernel runs ThinK's
                                      zero-filled attention from K_compact
"""
from rotatek_amd.baselines.recover import recover_spark, recover_think, selection_rotation
from rotatek_amd.baselines.spark import per_token_channel_prune, spark_prune
from rotatek_amd.baselines.think import think_score_and_compact

__all__ = ["think_score_and_compact", "per_token_channel_prune", "spark_prune", "recover_think",
           "recover_spark", "selection_rotation"]
