"""CPU oracle for the BlockFHT path — test infrastructure only.

``oracle.oracle`` is the numpy restatement (plus the torch-CPU port timed as
the CPU baseline); ``oracle.c_oracle`` binds the C restatement.  The product
package never imports anything from here.
"""
